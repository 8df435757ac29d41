// libadhip.so -- host runtime of the MI355X backend for the `ad` procedural
// IR: device/stream setup, the single-allocation arena, pinned staging for
// host transfers, hipRTC compilation, module loading, kernel launch and HIP
// graph capture/replay.  The C ABI is declared in include/adhip.h.
#include "../../include/adhip.h"

#include <hip/hip_runtime.h>
#include <hip/hiprtc.h>

#include "adhip_internal.h"

#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <vector>

namespace {

constexpr size_t kStageSlotBytes = 8u << 20;   // pinned staging: 8 slots x 8 MiB
constexpr int kStageSlots = 8;
constexpr int kEventSlots = 64;
constexpr int kTags = 4;                        // transfer-stream staging sets
constexpr int kFetchSets = 2;                   // transfer-stream device->host sets

thread_local std::string g_tls_error;

}  // namespace

struct adhip_module {
  hipModule_t mod = nullptr;
};

struct adhip_graph {
  hipGraph_t graph = nullptr;
  hipGraphExec_t exec = nullptr;
};

struct adhip_ctx {
  int device = 0;
  hipStream_t stream = nullptr;
  char* arena = nullptr;
  size_t arena_bytes = 0;
  char* stage = nullptr;                  // pinned host ring
  hipEvent_t stage_done[kStageSlots] = {};
  bool stage_used[kStageSlots] = {};
  int stage_next = 0;
  bool capturing = false;
  hipEvent_t events[kEventSlots] = {};
  // transfer stream for staged host->device copies overlapped with compute
  hipStream_t xfer = nullptr;
  struct Tag {
    char* host = nullptr;          // pinned staging of this set
    size_t cap = 0, used = 0;
    hipEvent_t copied = nullptr;   // on xfer: the set's copies are done
    hipEvent_t released = nullptr; // on stream: the set's device data is consumed
    bool copied_pending = false, released_pending = false, open = false;
  } tags[kTags];
  // device -> host copies on the transfer stream into pinned memory,
  // started after the compute stream's work so far
  struct Fetch {
    char* host = nullptr;          // pinned
    size_t cap = 0, used = 0;
    hipEvent_t ready = nullptr;    // on stream: the data to copy is complete
    hipEvent_t done = nullptr;     // on xfer: the set's copies are done
    bool open = false, pending = false;
  } fetches[kFetchSets];
  // extra compute streams and an event pool for launch graphs with
  // parallel branches (stream 0 is `stream`)
  std::vector<hipStream_t> lanes;
  std::vector<hipEvent_t> pool;
  std::vector<adhip_module*> modules;
  // device memory of library entry points that need scratch (grown on
  // demand), and this device's address of the static scratch array of the
  // entry points that allocate nothing
  void* ws = nullptr;
  size_t ws_bytes = 0;
  void* static_scratch = nullptr;
  std::string err;
};

namespace {

int fail(adhip_ctx* ctx, int code, const char* fmt, ...) {
  char buf[2048];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  if (ctx) ctx->err = buf; else g_tls_error = buf;
  return code;
}

#define HIP_TRY(ctx, call)                                                        \
  do {                                                                            \
    hipError_t e_ = (call);                                                       \
    if (e_ != hipSuccess)                                                         \
      return fail((ctx), (int)e_, "%s failed: %s", #call, hipGetErrorString(e_)); \
  } while (0)

int check_range(adhip_ctx* ctx, uint64_t off, size_t bytes) {
  if (!ctx->arena) return fail(ctx, ADHIP_E_STATE, "arena not reserved");
  if (off > ctx->arena_bytes || bytes > ctx->arena_bytes - off)
    return fail(ctx, ADHIP_E_ARG, "range [%llu, +%zu) outside arena of %zu bytes",
                (unsigned long long)off, bytes, ctx->arena_bytes);
  return 0;
}

}  // namespace

namespace adhip_internal {

hipStream_t stream_of(adhip_ctx* ctx) { return ctx->stream; }

int fail_arg(adhip_ctx* ctx, const char* fmt, ...) {
  char buf[2048];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  return fail(ctx, ADHIP_E_ARG, "%s", buf);
}

int fail_state(adhip_ctx* ctx, const char* fmt, ...) {
  char buf[2048];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  return fail(ctx, ADHIP_E_STATE, "%s", buf);
}

int fail_hip(adhip_ctx* ctx, hipError_t e, const char* what) {
  return fail(ctx, (int)e, "%s: %s", what, hipGetErrorString(e));
}

int workspace(adhip_ctx* ctx, size_t bytes, void** ptr) {
  if (bytes > ctx->ws_bytes) {
    if (ctx->capturing) return fail(ctx, ADHIP_E_STATE, "workspace of %zu bytes needed during graph capture", bytes);
    HIP_TRY(ctx, hipSetDevice(ctx->device));
    if (ctx->ws) {
      HIP_TRY(ctx, hipStreamSynchronize(ctx->stream));   // earlier calls may still read it
      HIP_TRY(ctx, hipFree(ctx->ws));
      ctx->ws = nullptr;
      ctx->ws_bytes = 0;
    }
    const size_t padded = (bytes + 255) & ~size_t(255);
    HIP_TRY(ctx, hipMalloc(&ctx->ws, padded));
    ctx->ws_bytes = padded;
  }
  *ptr = ctx->ws;
  return 0;
}

void* static_scratch(adhip_ctx* ctx) { return ctx->static_scratch; }

}  // namespace adhip_internal

extern "C" {

int adhip_create(int device, adhip_ctx** out) {
  if (!out) return fail(nullptr, ADHIP_E_ARG, "out is null");
  *out = nullptr;
  int n = 0;
  hipError_t e = hipGetDeviceCount(&n);
  if (e != hipSuccess) return fail(nullptr, (int)e, "hipGetDeviceCount: %s", hipGetErrorString(e));
  if (device < 0 || device >= n) return fail(nullptr, ADHIP_E_ARG, "device %d of %d", device, n);
  auto* ctx = new adhip_ctx();
  ctx->device = device;
  auto bail = [&](hipError_t err, const char* what) {
    g_tls_error = std::string(what) + ": " + hipGetErrorString(err);
    adhip_destroy(ctx);
    return (int)err;
  };
  if ((e = hipSetDevice(device)) != hipSuccess) return bail(e, "hipSetDevice");
  // this device's copy of the static scratch array (each device holds its
  // own, at its own address)
  if (int rc = adhip_internal::scratch_symbol(device, &ctx->static_scratch)) {
    g_tls_error = std::string("hipGetSymbolAddress(scratch): ") + hipGetErrorString((hipError_t)rc);
    adhip_destroy(ctx);
    return rc;
  }
  // default priority, non-blocking w.r.t. the legacy null stream
  if ((e = hipStreamCreateWithFlags(&ctx->stream, hipStreamNonBlocking)) != hipSuccess)
    return bail(e, "hipStreamCreate");
  if ((e = hipHostMalloc((void**)&ctx->stage, kStageSlotBytes * kStageSlots, hipHostMallocDefault)) != hipSuccess)
    return bail(e, "hipHostMalloc");
  for (int i = 0; i < kStageSlots; ++i)
    if ((e = hipEventCreateWithFlags(&ctx->stage_done[i], hipEventDisableTiming)) != hipSuccess)
      return bail(e, "hipEventCreate");
  *out = ctx;
  return 0;
}

void adhip_destroy(adhip_ctx* ctx) {
  if (!ctx) return;
  hipSetDevice(ctx->device);
  if (ctx->stream) hipStreamSynchronize(ctx->stream);
  for (auto* m : ctx->modules) {
    if (m->mod) hipModuleUnload(m->mod);
    delete m;
  }
  for (int i = 0; i < kEventSlots; ++i)
    if (ctx->events[i]) hipEventDestroy(ctx->events[i]);
  for (int i = 0; i < kStageSlots; ++i)
    if (ctx->stage_done[i]) hipEventDestroy(ctx->stage_done[i]);
  if (ctx->stage) hipHostFree(ctx->stage);
  if (ctx->xfer) hipStreamSynchronize(ctx->xfer);
  for (auto& t : ctx->tags) {
    if (t.copied) hipEventDestroy(t.copied);
    if (t.released) hipEventDestroy(t.released);
    if (t.host) hipHostFree(t.host);
  }
  for (auto& f : ctx->fetches) {
    if (f.ready) hipEventDestroy(f.ready);
    if (f.done) hipEventDestroy(f.done);
    if (f.host) hipHostFree(f.host);
  }
  if (ctx->xfer) hipStreamDestroy(ctx->xfer);
  for (auto st : ctx->lanes) {
    hipStreamSynchronize(st);
    hipStreamDestroy(st);
  }
  for (auto ev : ctx->pool) hipEventDestroy(ev);
  if (ctx->ws) hipFree(ctx->ws);
  if (ctx->arena) hipFree(ctx->arena);
  if (ctx->stream) hipStreamDestroy(ctx->stream);
  delete ctx;
}

const char* adhip_last_error(adhip_ctx* ctx) {
  return ctx ? ctx->err.c_str() : g_tls_error.c_str();
}

int adhip_device_info(adhip_ctx* ctx, int* num_cu, char* name, size_t name_cap) {
  if (!ctx) return fail(nullptr, ADHIP_E_ARG, "ctx is null");
  hipDeviceProp_t prop;
  HIP_TRY(ctx, hipGetDeviceProperties(&prop, ctx->device));
  if (num_cu) *num_cu = prop.multiProcessorCount;
  if (name && name_cap) {
    snprintf(name, name_cap, "%s (%s)", prop.name, prop.gcnArchName);
  }
  return 0;
}

int adhip_arena_reserve(adhip_ctx* ctx, size_t bytes, uint64_t* dev_base) {
  if (!ctx || !dev_base) return fail(ctx, ADHIP_E_ARG, "null argument");
  if (ctx->capturing) return fail(ctx, ADHIP_E_STATE, "arena_reserve during capture");
  HIP_TRY(ctx, hipSetDevice(ctx->device));
  if (ctx->arena) {
    HIP_TRY(ctx, hipStreamSynchronize(ctx->stream));
    if (ctx->xfer) HIP_TRY(ctx, hipStreamSynchronize(ctx->xfer));
    HIP_TRY(ctx, hipFree(ctx->arena));
    ctx->arena = nullptr;
    ctx->arena_bytes = 0;
  }
  size_t padded = (bytes + 255) & ~size_t(255);
  if (padded == 0) padded = 256;
  HIP_TRY(ctx, hipMalloc((void**)&ctx->arena, padded));
  HIP_TRY(ctx, hipMemsetAsync(ctx->arena, 0, padded, ctx->stream));
  HIP_TRY(ctx, hipStreamSynchronize(ctx->stream));
  ctx->arena_bytes = padded;
  *dev_base = (uint64_t)(uintptr_t)ctx->arena;
  return 0;
}

int adhip_write(adhip_ctx* ctx, uint64_t dst_off, const void* host, size_t bytes) {
  if (!ctx || (!host && bytes)) return fail(ctx, ADHIP_E_ARG, "null argument");
  if (ctx->capturing) return fail(ctx, ADHIP_E_STATE, "host write during graph capture");
  if (int r = check_range(ctx, dst_off, bytes)) return r;
  const char* src = static_cast<const char*>(host);
  size_t done = 0;
  while (done < bytes) {
    const int slot = ctx->stage_next;
    ctx->stage_next = (slot + 1) % kStageSlots;
    if (ctx->stage_used[slot]) HIP_TRY(ctx, hipEventSynchronize(ctx->stage_done[slot]));
    const size_t n = (bytes - done < kStageSlotBytes) ? bytes - done : kStageSlotBytes;
    char* staged = ctx->stage + (size_t)slot * kStageSlotBytes;
    std::memcpy(staged, src + done, n);
    HIP_TRY(ctx, hipMemcpyAsync(ctx->arena + dst_off + done, staged, n, hipMemcpyHostToDevice, ctx->stream));
    HIP_TRY(ctx, hipEventRecord(ctx->stage_done[slot], ctx->stream));
    ctx->stage_used[slot] = true;
    done += n;
  }
  return 0;
}

int adhip_stage_begin(adhip_ctx* ctx, int tag) {
  if (!ctx || tag < 0 || tag >= kTags) return fail(ctx, ADHIP_E_ARG, "bad staging set %d", tag);
  if (ctx->capturing) return fail(ctx, ADHIP_E_STATE, "staged copies during graph capture");
  auto& t = ctx->tags[tag];
  if (t.open) return fail(ctx, ADHIP_E_STATE, "staging set %d already open", tag);
  HIP_TRY(ctx, hipSetDevice(ctx->device));
  if (!ctx->xfer) HIP_TRY(ctx, hipStreamCreateWithFlags(&ctx->xfer, hipStreamNonBlocking));
  if (!t.copied) HIP_TRY(ctx, hipEventCreateWithFlags(&t.copied, hipEventDisableTiming));
  if (!t.released) HIP_TRY(ctx, hipEventCreateWithFlags(&t.released, hipEventDisableTiming));
  // the pinned buffer is reused: its previous copies must have left it
  if (t.copied_pending) HIP_TRY(ctx, hipEventSynchronize(t.copied));
  t.copied_pending = false;
  // the device data of this set is rewritten: its previous readers must be done
  if (t.released_pending) HIP_TRY(ctx, hipStreamWaitEvent(ctx->xfer, t.released, 0));
  t.used = 0;
  t.open = true;
  return 0;
}

int adhip_stage_write(adhip_ctx* ctx, int tag, uint64_t dst_off, const void* host, size_t bytes) {
  if (!ctx || tag < 0 || tag >= kTags || (!host && bytes)) return fail(ctx, ADHIP_E_ARG, "bad argument");
  auto& t = ctx->tags[tag];
  if (!t.open) return fail(ctx, ADHIP_E_STATE, "staging set %d not open", tag);
  if (int r = check_range(ctx, dst_off, bytes)) return r;
  const size_t need = t.used + ((bytes + 255) & ~size_t(255));
  if (need > t.cap) {
    // nothing of this set is in flight (stage_begin waited), so it may move
    char* bigger = nullptr;
    const size_t cap = need > 2 * t.cap ? need : 2 * t.cap;
    HIP_TRY(ctx, hipHostMalloc((void**)&bigger, cap, hipHostMallocDefault));
    if (t.host) {
      HIP_TRY(ctx, hipStreamSynchronize(ctx->xfer));   // copies of this round read the old buffer
      std::memcpy(bigger, t.host, t.used);
      hipHostFree(t.host);
    }
    t.host = bigger;
    t.cap = cap;
  }
  char* staged = t.host + t.used;
  std::memcpy(staged, host, bytes);
  HIP_TRY(ctx, hipMemcpyAsync(ctx->arena + dst_off, staged, bytes, hipMemcpyHostToDevice, ctx->xfer));
  t.used = need;
  return 0;
}

int adhip_stage_end(adhip_ctx* ctx, int tag) {
  if (!ctx || tag < 0 || tag >= kTags) return fail(ctx, ADHIP_E_ARG, "bad staging set %d", tag);
  auto& t = ctx->tags[tag];
  if (!t.open) return fail(ctx, ADHIP_E_STATE, "staging set %d not open", tag);
  HIP_TRY(ctx, hipEventRecord(t.copied, ctx->xfer));
  HIP_TRY(ctx, hipStreamWaitEvent(ctx->stream, t.copied, 0));
  t.copied_pending = true;
  t.open = false;
  return 0;
}

int adhip_stage_release(adhip_ctx* ctx, int tag) {
  if (!ctx || tag < 0 || tag >= kTags) return fail(ctx, ADHIP_E_ARG, "bad staging set %d", tag);
  auto& t = ctx->tags[tag];
  if (!t.released) return fail(ctx, ADHIP_E_STATE, "staging set %d never used", tag);
  HIP_TRY(ctx, hipEventRecord(t.released, ctx->stream));
  t.released_pending = true;
  return 0;
}

int adhip_fetch_reserve(adhip_ctx* ctx, int set, size_t bytes) {
  if (!ctx || set < 0 || set >= kFetchSets) return fail(ctx, ADHIP_E_ARG, "bad fetch set %d", set);
  auto& f = ctx->fetches[set];
  if (f.open || f.pending) return fail(ctx, ADHIP_E_STATE, "fetch set %d in use", set);
  HIP_TRY(ctx, hipSetDevice(ctx->device));
  if (!ctx->xfer) HIP_TRY(ctx, hipStreamCreateWithFlags(&ctx->xfer, hipStreamNonBlocking));
  if (!f.ready) HIP_TRY(ctx, hipEventCreateWithFlags(&f.ready, hipEventDisableTiming));
  if (!f.done) HIP_TRY(ctx, hipEventCreateWithFlags(&f.done, hipEventDisableTiming));
  if (bytes > f.cap) {
    if (f.host) HIP_TRY(ctx, hipHostFree(f.host));
    f.host = nullptr;
    f.cap = 0;
    HIP_TRY(ctx, hipHostMalloc((void**)&f.host, bytes, hipHostMallocDefault));
    f.cap = bytes;
  }
  return 0;
}

int adhip_fetch_begin(adhip_ctx* ctx, int set) {
  if (!ctx || set < 0 || set >= kFetchSets) return fail(ctx, ADHIP_E_ARG, "bad fetch set %d", set);
  if (ctx->capturing) return fail(ctx, ADHIP_E_STATE, "fetch during graph capture");
  auto& f = ctx->fetches[set];
  if (!f.ready) return fail(ctx, ADHIP_E_STATE, "fetch set %d not reserved", set);
  if (f.open || f.pending) return fail(ctx, ADHIP_E_STATE, "fetch set %d not taken yet", set);
  HIP_TRY(ctx, hipEventRecord(f.ready, ctx->stream));
  HIP_TRY(ctx, hipStreamWaitEvent(ctx->xfer, f.ready, 0));
  f.used = 0;
  f.open = true;
  return 0;
}

int adhip_fetch_copy(adhip_ctx* ctx, int set, uint64_t src_off, size_t bytes, size_t* host_off) {
  if (!ctx || set < 0 || set >= kFetchSets || !host_off) return fail(ctx, ADHIP_E_ARG, "bad argument");
  auto& f = ctx->fetches[set];
  if (!f.open) return fail(ctx, ADHIP_E_STATE, "fetch set %d not open", set);
  if (int r = check_range(ctx, src_off, bytes)) return r;
  const size_t need = f.used + ((bytes + 255) & ~size_t(255));
  if (need > f.cap) return fail(ctx, ADHIP_E_ARG, "fetch set %d: %zu bytes reserved, %zu needed", set, f.cap, need);
  if (bytes) HIP_TRY(ctx, hipMemcpyAsync(f.host + f.used, ctx->arena + src_off, bytes, hipMemcpyDeviceToHost, ctx->xfer));
  *host_off = f.used;
  f.used = need;
  return 0;
}

int adhip_fetch_end(adhip_ctx* ctx, int set) {
  if (!ctx || set < 0 || set >= kFetchSets) return fail(ctx, ADHIP_E_ARG, "bad fetch set %d", set);
  auto& f = ctx->fetches[set];
  if (!f.open) return fail(ctx, ADHIP_E_STATE, "fetch set %d not open", set);
  HIP_TRY(ctx, hipEventRecord(f.done, ctx->xfer));
  f.open = false;
  f.pending = true;
  return 0;
}

int adhip_fetch_take(adhip_ctx* ctx, int set, size_t host_off, void* dst, size_t bytes) {
  if (!ctx || set < 0 || set >= kFetchSets || (!dst && bytes)) return fail(ctx, ADHIP_E_ARG, "bad argument");
  auto& f = ctx->fetches[set];
  if (f.open) return fail(ctx, ADHIP_E_STATE, "fetch set %d still open", set);
  if (host_off > f.used || bytes > f.used - host_off) return fail(ctx, ADHIP_E_ARG, "fetch set %d: range out of bounds", set);
  if (f.pending) {
    HIP_TRY(ctx, hipEventSynchronize(f.done));
    f.pending = false;
  }
  if (bytes) std::memcpy(dst, f.host + host_off, bytes);
  return 0;
}

int adhip_read(adhip_ctx* ctx, uint64_t src_off, void* host, size_t bytes) {
  if (!ctx || (!host && bytes)) return fail(ctx, ADHIP_E_ARG, "null argument");
  if (ctx->capturing) return fail(ctx, ADHIP_E_STATE, "host read during graph capture");
  if (int r = check_range(ctx, src_off, bytes)) return r;
  char* dst = static_cast<char*>(host);
  // every staging slot is free once the stream drains
  HIP_TRY(ctx, hipStreamSynchronize(ctx->stream));
  size_t done = 0;
  while (done < bytes) {
    const size_t n = (bytes - done < kStageSlotBytes) ? bytes - done : kStageSlotBytes;
    HIP_TRY(ctx, hipMemcpyAsync(ctx->stage, ctx->arena + src_off + done, n, hipMemcpyDeviceToHost, ctx->stream));
    HIP_TRY(ctx, hipStreamSynchronize(ctx->stream));
    std::memcpy(dst + done, ctx->stage, n);
    done += n;
  }
  return 0;
}

int adhip_copy(adhip_ctx* ctx, uint64_t dst_off, uint64_t src_off, size_t bytes) {
  if (!ctx) return fail(ctx, ADHIP_E_ARG, "null ctx");
  if (int r = check_range(ctx, dst_off, bytes)) return r;
  if (int r = check_range(ctx, src_off, bytes)) return r;
  if (bytes == 0) return 0;
  HIP_TRY(ctx, hipMemcpyAsync(ctx->arena + dst_off, ctx->arena + src_off, bytes,
                              hipMemcpyDeviceToDevice, ctx->stream));
  return 0;
}

int adhip_compile(const char* src, const char* options, void** code, size_t* code_size,
                  char* log, size_t log_cap) {
  if (!src || !code || !code_size) return fail(nullptr, ADHIP_E_ARG, "null argument");
  *code = nullptr;
  *code_size = 0;
  if (log && log_cap) log[0] = 0;
  std::vector<std::string> opts;
  if (options) {
    const char* p = options;
    while (*p) {
      while (*p == ' ') ++p;
      const char* q = p;
      while (*q && *q != ' ') ++q;
      if (q > p) opts.emplace_back(p, q - p);
      p = q;
    }
  }
  std::vector<const char*> argv;
  for (auto& o : opts) argv.push_back(o.c_str());
  hiprtcProgram prog;
  hiprtcResult r = hiprtcCreateProgram(&prog, src, "adhip_kernel.hip", 0, nullptr, nullptr);
  if (r != HIPRTC_SUCCESS) return fail(nullptr, (int)r, "hiprtcCreateProgram: %s", hiprtcGetErrorString(r));
  r = hiprtcCompileProgram(prog, (int)argv.size(), argv.data());
  size_t lsz = 0;
  hiprtcGetProgramLogSize(prog, &lsz);
  if (log && log_cap && lsz > 1) {
    std::vector<char> buf(lsz + 1, 0);
    hiprtcGetProgramLog(prog, buf.data());
    snprintf(log, log_cap, "%s", buf.data());
  }
  if (r != HIPRTC_SUCCESS) {
    hiprtcDestroyProgram(&prog);
    return fail(nullptr, ADHIP_E_COMPILE, "hipRTC compile failed: %s", hiprtcGetErrorString(r));
  }
  size_t sz = 0;
  hiprtcGetCodeSize(prog, &sz);
  void* buf = std::malloc(sz ? sz : 1);
  if (!buf) {
    hiprtcDestroyProgram(&prog);
    return fail(nullptr, ADHIP_E_ARG, "out of host memory");
  }
  hiprtcGetCode(prog, static_cast<char*>(buf));
  hiprtcDestroyProgram(&prog);
  *code = buf;
  *code_size = sz;
  return 0;
}

void adhip_free(void* p) { std::free(p); }

int adhip_module_load(adhip_ctx* ctx, const void* code, size_t code_size, adhip_module** out) {
  if (!ctx || !code || !code_size || !out) return fail(ctx, ADHIP_E_ARG, "null argument");
  HIP_TRY(ctx, hipSetDevice(ctx->device));
  auto* m = new adhip_module();
  hipError_t e = hipModuleLoadData(&m->mod, code);
  if (e != hipSuccess) {
    delete m;
    return fail(ctx, (int)e, "hipModuleLoadData: %s", hipGetErrorString(e));
  }
  ctx->modules.push_back(m);
  *out = m;
  return 0;
}

int adhip_module_function(adhip_module* mod, const char* name, void** fn) {
  if (!mod || !name || !fn) return fail(nullptr, ADHIP_E_ARG, "null argument");
  hipFunction_t f = nullptr;
  hipError_t e = hipModuleGetFunction(&f, mod->mod, name);
  if (e != hipSuccess) return fail(nullptr, ADHIP_E_NOTFOUND, "kernel %s: %s", name, hipGetErrorString(e));
  *fn = (void*)f;
  return 0;
}

int adhip_launch(adhip_ctx* ctx, void* fn, const uint32_t grid[3], const uint32_t block[3],
                 uint32_t shared_bytes, const uint64_t* args, size_t nargs) {
  if (!ctx || !fn || !grid || !block || (nargs && !args)) return fail(ctx, ADHIP_E_ARG, "null argument");
  if (grid[0] == 0 || grid[1] == 0 || grid[2] == 0) return 0;   // empty NDRange
  if (block[0] * block[1] * block[2] > 1024) return fail(ctx, ADHIP_E_ARG, "block too large");
  void* params[64];
  if (nargs > 64) return fail(ctx, ADHIP_E_ARG, "too many kernel arguments (%zu)", nargs);
  for (size_t i = 0; i < nargs; ++i) params[i] = (void*)(args + i);
  HIP_TRY(ctx, hipModuleLaunchKernel((hipFunction_t)fn, grid[0], grid[1], grid[2], block[0], block[1],
                                     block[2], shared_bytes, ctx->stream, params, nullptr));
  return 0;
}

namespace {
hipStream_t lane(adhip_ctx* ctx, int s) {
  if (s == 0) return ctx->stream;
  if (s < 0 || s > (int)ctx->lanes.size()) return nullptr;
  return ctx->lanes[s - 1];
}
}  // namespace

int adhip_lanes_reserve(adhip_ctx* ctx, int streams, int events) {
  if (!ctx || streams < 1 || events < 0) return fail(ctx, ADHIP_E_ARG, "bad argument");
  if (ctx->capturing) return fail(ctx, ADHIP_E_STATE, "lanes_reserve during capture");
  HIP_TRY(ctx, hipSetDevice(ctx->device));
  while ((int)ctx->lanes.size() < streams - 1) {
    hipStream_t st = nullptr;   // default priority
    HIP_TRY(ctx, hipStreamCreateWithFlags(&st, hipStreamNonBlocking));
    ctx->lanes.push_back(st);
  }
  while ((int)ctx->pool.size() < events) {
    hipEvent_t ev = nullptr;
    HIP_TRY(ctx, hipEventCreateWithFlags(&ev, hipEventDisableTiming));
    ctx->pool.push_back(ev);
  }
  return 0;
}

int adhip_launch_on(adhip_ctx* ctx, int s, void* fn, const uint32_t grid[3], const uint32_t block[3],
                    uint32_t shared_bytes, const uint64_t* args, size_t nargs) {
  if (!ctx || !fn || !grid || !block || (nargs && !args)) return fail(ctx, ADHIP_E_ARG, "null argument");
  hipStream_t st = lane(ctx, s);
  if (!st) return fail(ctx, ADHIP_E_ARG, "no stream %d", s);
  if (grid[0] == 0 || grid[1] == 0 || grid[2] == 0) return 0;
  if (block[0] * block[1] * block[2] > 1024) return fail(ctx, ADHIP_E_ARG, "block too large");
  void* params[64];
  if (nargs > 64) return fail(ctx, ADHIP_E_ARG, "too many kernel arguments (%zu)", nargs);
  for (size_t i = 0; i < nargs; ++i) params[i] = (void*)(args + i);
  HIP_TRY(ctx, hipModuleLaunchKernel((hipFunction_t)fn, grid[0], grid[1], grid[2], block[0], block[1],
                                     block[2], shared_bytes, st, params, nullptr));
  return 0;
}

int adhip_record_on(adhip_ctx* ctx, int s, int ev) {
  if (!ctx) return fail(ctx, ADHIP_E_ARG, "null ctx");
  hipStream_t st = lane(ctx, s);
  if (!st || ev < 0 || ev >= (int)ctx->pool.size()) return fail(ctx, ADHIP_E_ARG, "bad stream %d / event %d", s, ev);
  HIP_TRY(ctx, hipEventRecord(ctx->pool[ev], st));
  return 0;
}

int adhip_wait_on(adhip_ctx* ctx, int s, int ev) {
  if (!ctx) return fail(ctx, ADHIP_E_ARG, "null ctx");
  hipStream_t st = lane(ctx, s);
  if (!st || ev < 0 || ev >= (int)ctx->pool.size()) return fail(ctx, ADHIP_E_ARG, "bad stream %d / event %d", s, ev);
  HIP_TRY(ctx, hipStreamWaitEvent(st, ctx->pool[ev], 0));
  return 0;
}

int adhip_graph_begin(adhip_ctx* ctx) {
  if (!ctx) return fail(ctx, ADHIP_E_ARG, "null ctx");
  if (ctx->capturing) return fail(ctx, ADHIP_E_STATE, "already capturing");
  HIP_TRY(ctx, hipStreamBeginCapture(ctx->stream, hipStreamCaptureModeThreadLocal));
  ctx->capturing = true;
  return 0;
}

int adhip_graph_end(adhip_ctx* ctx, adhip_graph** out) {
  if (!ctx || !out) return fail(ctx, ADHIP_E_ARG, "null argument");
  if (!ctx->capturing) return fail(ctx, ADHIP_E_STATE, "not capturing");
  ctx->capturing = false;
  auto* g = new adhip_graph();
  hipError_t e = hipStreamEndCapture(ctx->stream, &g->graph);
  if (e != hipSuccess) {
    delete g;
    return fail(ctx, (int)e, "hipStreamEndCapture: %s", hipGetErrorString(e));
  }
  e = hipGraphInstantiate(&g->exec, g->graph, nullptr, nullptr, 0);
  if (e != hipSuccess) {
    hipGraphDestroy(g->graph);
    delete g;
    return fail(ctx, (int)e, "hipGraphInstantiate: %s", hipGetErrorString(e));
  }
  *out = g;
  return 0;
}

int adhip_graph_end_dag(adhip_ctx* ctx, int32_t n_nodes, const int32_t* dep_offsets, const int32_t* deps,
                        adhip_graph** out) {
  if (!ctx || !out || n_nodes < 0 || (n_nodes && !dep_offsets)) return fail(ctx, ADHIP_E_ARG, "bad argument");
  if (!ctx->capturing) return fail(ctx, ADHIP_E_STATE, "not capturing");
  ctx->capturing = false;
  hipGraph_t graph = nullptr;
  HIP_TRY(ctx, hipStreamEndCapture(ctx->stream, &graph));
  auto drop = [&](int code, const char* fmt, auto... a) {
    hipGraphDestroy(graph);
    return fail(ctx, code, fmt, a...);
  };
  // the captured work is a chain: walk it from its root in capture order
  std::vector<hipGraphNode_t> order;
  size_t nroots = 0;
  hipError_t e = hipGraphGetRootNodes(graph, nullptr, &nroots);
  if (e != hipSuccess) return drop((int)e, "hipGraphGetRootNodes: %s", hipGetErrorString(e));
  if (nroots > 1) return drop(ADHIP_E_STATE, "captured graph has %zu roots, expected a chain", nroots);
  if (nroots == 1) {
    hipGraphNode_t cur = nullptr;
    e = hipGraphGetRootNodes(graph, &cur, &nroots);
    if (e != hipSuccess) return drop((int)e, "hipGraphGetRootNodes: %s", hipGetErrorString(e));
    while (true) {
      order.push_back(cur);
      size_t nnext = 0;
      e = hipGraphNodeGetDependentNodes(cur, nullptr, &nnext);
      if (e != hipSuccess) return drop((int)e, "hipGraphNodeGetDependentNodes: %s", hipGetErrorString(e));
      if (nnext == 0) break;
      if (nnext > 1) return drop(ADHIP_E_STATE, "captured node %zu has %zu successors, expected a chain",
                                 order.size() - 1, nnext);
      hipGraphNode_t next = nullptr;
      e = hipGraphNodeGetDependentNodes(cur, &next, &nnext);
      if (e != hipSuccess) return drop((int)e, "hipGraphNodeGetDependentNodes: %s", hipGetErrorString(e));
      cur = next;
    }
  }
  if ((int64_t)order.size() != n_nodes)
    return drop(ADHIP_E_ARG, "captured %zu graph nodes, the dependency lists describe %d", order.size(), n_nodes);
  // replace the chain edges by the given dependencies
  std::vector<hipGraphNode_t> from, to;
  for (size_t i = 1; i < order.size(); ++i) {
    from.push_back(order[i - 1]);
    to.push_back(order[i]);
  }
  if (!from.empty()) {
    e = hipGraphRemoveDependencies(graph, from.data(), to.data(), from.size());
    if (e != hipSuccess) return drop((int)e, "hipGraphRemoveDependencies: %s", hipGetErrorString(e));
  }
  from.clear();
  to.clear();
  for (int32_t i = 0; i < n_nodes; ++i) {
    for (int32_t k = dep_offsets[i]; k < dep_offsets[i + 1]; ++k) {
      const int32_t d = deps[k];
      if (d < 0 || d >= i) return drop(ADHIP_E_ARG, "node %d depends on node %d (must be an earlier node)", i, d);
      from.push_back(order[d]);
      to.push_back(order[i]);
    }
  }
  if (!from.empty()) {
    e = hipGraphAddDependencies(graph, from.data(), to.data(), from.size());
    if (e != hipSuccess) return drop((int)e, "hipGraphAddDependencies: %s", hipGetErrorString(e));
  }
  auto* g = new adhip_graph();
  g->graph = graph;
  e = hipGraphInstantiate(&g->exec, g->graph, nullptr, nullptr, 0);
  if (e != hipSuccess) {
    hipGraphDestroy(g->graph);
    delete g;
    return fail(ctx, (int)e, "hipGraphInstantiate: %s", hipGetErrorString(e));
  }
  *out = g;
  return 0;
}

int adhip_graph_launch(adhip_ctx* ctx, adhip_graph* g) {
  if (!ctx || !g) return fail(ctx, ADHIP_E_ARG, "null argument");
  HIP_TRY(ctx, hipGraphLaunch(g->exec, ctx->stream));
  return 0;
}

void adhip_graph_destroy(adhip_graph* g) {
  if (!g) return;
  if (g->exec) hipGraphExecDestroy(g->exec);
  if (g->graph) hipGraphDestroy(g->graph);
  delete g;
}

int adhip_sync(adhip_ctx* ctx) {
  if (!ctx) return fail(ctx, ADHIP_E_ARG, "null ctx");
  HIP_TRY(ctx, hipStreamSynchronize(ctx->stream));
  if (ctx->xfer) HIP_TRY(ctx, hipStreamSynchronize(ctx->xfer));
  return 0;
}

int adhip_event_record(adhip_ctx* ctx, int slot) {
  if (!ctx || slot < 0 || slot >= kEventSlots) return fail(ctx, ADHIP_E_ARG, "bad event slot %d", slot);
  if (!ctx->events[slot]) HIP_TRY(ctx, hipEventCreate(&ctx->events[slot]));
  HIP_TRY(ctx, hipEventRecord(ctx->events[slot], ctx->stream));
  return 0;
}

int adhip_event_elapsed(adhip_ctx* ctx, int a, int b, float* ms) {
  if (!ctx || !ms || a < 0 || b < 0 || a >= kEventSlots || b >= kEventSlots || !ctx->events[a] ||
      !ctx->events[b])
    return fail(ctx, ADHIP_E_ARG, "bad event slots %d %d", a, b);
  HIP_TRY(ctx, hipEventSynchronize(ctx->events[b]));
  HIP_TRY(ctx, hipEventElapsedTime(ms, ctx->events[a], ctx->events[b]));
  return 0;
}

}  // extern "C"
