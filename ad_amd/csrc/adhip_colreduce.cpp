// Column reduction of a row-major [rows, cols] fp32 matrix on caller device
// memory: out[c] = SUM or MAX over r of x[r * cols + c].  The rows are split
// into chunks over blocks (the same policy as the generated column
// reductions: chunks double until there are 512 blocks, at most 128 chunks,
// at least 64 rows each); each chunk's result goes to a scratch row
// [chunk][cols], and a second kernel combines the chunks in chunk order.
//
// Two entry points share the kernels and differ only in where the scratch
// rows live:
//  * adhip_reduce_cols: device memory the context allocates on first need
//    and keeps (grown when a call needs more) until adhip_destroy;
//  * adhip_reduce_cols_noalloc: the file-scope `scratch` array below, whose
//    per-device address is looked up once per device (hipGetSymbolAddress at
//    the context's creation); it allocates nothing, so code under graph
//    capture or a loop that must not allocate can call it.  Every call on
//    one GPU shares that GPU's array: calls that overlap on one GPU (other
//    streams, other contexts or threads) race.  Every scratch element a
//    call reads was written by the same call, so nothing needs clearing.
#include "../../include/adhip.h"

#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstring>
#include <map>
#include <mutex>

#include "adhip_kernels.h"
#include "adhip_internal.h"

namespace {

constexpr size_t kScratchFloats = ADHIP_REDUCE_COLS_SCRATCH_FLOATS;
static __device__ __align__(256) float scratch[kScratchFloats];

template <bool V4>
struct ColLoad {
  static constexpr bool kVec = false;
  static constexpr bool kVecX = V4;
  const float* x;
  unsigned cols;
  __device__ float at(unsigned c, unsigned r) const { return x[(size_t)r * cols + c]; }
  __device__ float4 at4(unsigned c, unsigned r) const {
    return *reinterpret_cast<const float4*>(x + (size_t)r * cols + c);
  }
  __device__ bool inc(unsigned) const { return true; }
};

struct ToRow {          // chunk results: row `chunk` of [chunks][cols]
  float* dst;
  unsigned cols;
  __device__ void operator()(float v, unsigned c, int chunk) const { dst[(size_t)chunk * cols + c] = v; }
};

template <int OP, int SPLIT, bool V4>
__global__ void __launch_bounds__(256) colreduce_chunks(const float* x, float* dst, unsigned rows, unsigned cols) {
  adhip::reduce_cols<OP, SPLIT>(ColLoad<V4>{x, cols}, ToRow{dst, cols}, cols, rows, false);
}

template <int OP>
__global__ void __launch_bounds__(256) colreduce_combine(const float* part, float* out, unsigned chunks, unsigned cols) {
  const unsigned c = blockIdx.x * 256 + threadIdx.x;
  if (c >= cols) return;
  float a = part[c];
  for (unsigned s = 1; s < chunks; ++s) a = adhip::rop<OP>(a, part[(size_t)s * cols + c]);
  out[c] = a;
}

unsigned split_for(unsigned rows, unsigned cols) {
  const unsigned blocks = (cols + 63) / 64;
  unsigned split = 1;
  while (blocks * split < 512 && split < 128 && rows / (2 * split) >= 64) split *= 2;
  return split;
}

template <int OP, bool V4>
hipError_t launch_chunks(unsigned split, const float* x, float* dst, unsigned rows, unsigned cols, hipStream_t st) {
  const dim3 grid((cols + 63) / 64, split, 1);
  switch (split) {
#define ADHIP_CASE(S) \
  case S: colreduce_chunks<OP, S, V4><<<grid, 256, 0, st>>>(x, dst, rows, cols); break;
    ADHIP_CASE(1) ADHIP_CASE(2) ADHIP_CASE(4) ADHIP_CASE(8) ADHIP_CASE(16) ADHIP_CASE(32) ADHIP_CASE(64)
    ADHIP_CASE(128)
#undef ADHIP_CASE
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

// Validates, then enqueues the chunk pass (into `part`, or straight into
// `out` when there is one chunk) and the combine pass on the context's stream.
int enqueue(adhip_ctx* ctx, const float* x, float* out, uint32_t rows, uint32_t cols, int op, float* part,
            unsigned split) {
  hipStream_t st = adhip_internal::stream_of(ctx);
  const bool v4 = cols % 4 == 0 && (reinterpret_cast<uintptr_t>(x) & 15) == 0;
  float* dst = split == 1 ? out : part;
  hipError_t e;
  if (op == 0)
    e = v4 ? launch_chunks<0, true>(split, x, dst, rows, cols, st) : launch_chunks<0, false>(split, x, dst, rows, cols, st);
  else
    e = v4 ? launch_chunks<1, true>(split, x, dst, rows, cols, st) : launch_chunks<1, false>(split, x, dst, rows, cols, st);
  if (e != hipSuccess) return adhip_internal::fail_hip(ctx, e, "column reduction chunk pass");
  if (split > 1) {
    const dim3 grid((cols + 255) / 256, 1, 1);
    if (op == 0) colreduce_combine<0><<<grid, 256, 0, st>>>(part, out, split, cols);
    else colreduce_combine<1><<<grid, 256, 0, st>>>(part, out, split, cols);
    e = hipGetLastError();
    if (e != hipSuccess) return adhip_internal::fail_hip(ctx, e, "column reduction combine pass");
  }
  return 0;
}

int check_args(adhip_ctx* ctx, const float* x, float* out, uint32_t rows, uint32_t cols, int op) {
  if (!ctx) return adhip_internal::fail_arg(nullptr, "ctx is null");
  if (op != 0 && op != 1) return adhip_internal::fail_arg(ctx, "op must be 0 (SUM) or 1 (MAX), got %d", op);
  if (cols && (!x || !out)) return adhip_internal::fail_arg(ctx, "null input or output pointer");
  if (cols && rows == 0) return adhip_internal::fail_arg(ctx, "a reduction over 0 rows has no value");
  if ((uint64_t)rows * cols > (1ull << 32)) return adhip_internal::fail_arg(ctx, "rows x cols above 2^32 elements");
  return 0;
}

}  // namespace

namespace adhip_internal {
// The address of `scratch` on `device`, which must be current: looked up
// once per device (hipGetSymbolAddress; each device holds its own copy of
// the array, at its own address) and kept until the process ends.  Called
// from adhip_create.
int scratch_symbol(int device, void** ptr) {
  static std::mutex lock;
  static std::map<int, void*> by_device;
  std::lock_guard<std::mutex> hold(lock);
  auto it = by_device.find(device);
  if (it == by_device.end()) {
    void* p = nullptr;
    hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return (int)e;
    it = by_device.emplace(device, p).first;
  }
  *ptr = it->second;
  return 0;
}
}  // namespace adhip_internal

extern "C" {

int adhip_reduce_cols(adhip_ctx* ctx, const float* x, float* out, uint32_t rows, uint32_t cols, int op) {
  if (int r = check_args(ctx, x, out, rows, cols, op)) return r;
  if (cols == 0) return 0;
  const unsigned split = split_for(rows, cols);
  float* part = nullptr;
  if (split > 1) {
    if (int rc = adhip_internal::workspace(ctx, (size_t)split * cols * sizeof(float), (void**)&part)) return rc;
  }
  return enqueue(ctx, x, out, rows, cols, op, part, split);
}

int adhip_reduce_cols_noalloc(adhip_ctx* ctx, const float* x, float* out, uint32_t rows, uint32_t cols, int op) {
  if (int r = check_args(ctx, x, out, rows, cols, op)) return r;
  if (cols == 0) return 0;
  const unsigned split = split_for(rows, cols);
  if ((size_t)split * cols > kScratchFloats)
    return adhip_internal::fail_arg(ctx, "adhip_reduce_cols_noalloc: %u chunks x %u columns need %zu scratch floats, "
                                         "the static scratch holds %zu", split, cols, (size_t)split * cols,
                                    kScratchFloats);
  float* part = nullptr;
  if (split > 1) {
    part = static_cast<float*>(adhip_internal::static_scratch(ctx));
    if (!part) return adhip_internal::fail_state(ctx, "static scratch address unknown on this device");
  }
  return enqueue(ctx, x, out, rows, cols, op, part, split);
}

}  // extern "C"
