/*
 * adhip.h -- C ABI of libadhip.so, the MI355X execution backend for the
 * procedural IR of the `ad` autodiff compiler.
 *
 * The reference backend reaches its device through ctypes bindings of the
 * OpenCL C API (autodiff/device/opencl/cl_helper.py).  Each entry point
 * below replaces the OpenCL calls named beside it; the Python backend
 * (ad_amd/device/hip) binds these with ctypes the same way.
 *
 * Conventions: every int-returning call returns 0 on success, otherwise a
 * hipError_t / hiprtcResult value or one of the ADHIP_E_* codes, and the
 * message is available from adhip_last_error().  One context per process
 * and thread; all device work of a context is ordered on one HIP stream.
 * No PyTorch or other framework types cross this boundary.
 */
#ifndef ADHIP_H
#define ADHIP_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct adhip_ctx adhip_ctx;
typedef struct adhip_module adhip_module;
typedef struct adhip_graph adhip_graph;

#define ADHIP_E_ARG      1001  /* bad argument (null pointer, size, range) */
#define ADHIP_E_STATE    1002  /* call not valid in the current state */
#define ADHIP_E_COMPILE  1003  /* hipRTC compile failed; log returned */
#define ADHIP_E_NOTFOUND 1004  /* kernel symbol not found in module */

/* Size of the static scratch array of the column reduction's variant that
 * allocates nothing: 2^18 floats (1 MiB) per device, held until the process
 * ends. */
#define ADHIP_REDUCE_COLS_SCRATCH_FLOATS (1u << 18)

/* Device + stream + pinned staging.  Replaces clGetPlatformIDs /
 * clGetDeviceIDs / clCreateContext / clCreateCommandQueue
 * (cl_helper.py:36-139, device.py:16-51). */
int  adhip_create(int device, adhip_ctx** out);
/* Frees everything the context owns.  Replaces clReleaseMemObject /
 * clReleaseKernel / clReleaseCommandQueue / clReleaseContext
 * (cl_helper.py:140-175, device.py:139-153). */
void adhip_destroy(adhip_ctx* ctx);
/* Message of the last failing call on this context (thread-local when
 * ctx is NULL). */
const char* adhip_last_error(adhip_ctx* ctx);
/* Number of compute units and device name, for launch sizing and logs. */
int  adhip_device_info(adhip_ctx* ctx, int* num_cu, char* name, size_t name_cap);

/* One hipMalloc holding every buffer of a Proc (the tetris arena, each
 * Tensor, the hoisted leftovers) plus scratch; zero-filled.  Replaces one
 * clCreateBuffer per AllocEntry (cl_helper.py:151-170). */
int  adhip_arena_reserve(adhip_ctx* ctx, size_t bytes, uint64_t* dev_base);

/* Stream-ordered host -> device copy of `bytes` into arena byte offset
 * `dst_off`.  The host buffer is copied to pinned staging before the call
 * returns, so it is only borrowed for the call.  Replaces
 * clEnqueueWriteBuffer (cl_helper.py:304-332). */
int  adhip_write(adhip_ctx* ctx, uint64_t dst_off, const void* host, size_t bytes);
/* Blocking device -> host copy after all queued work.  Replaces
 * clEnqueueReadBuffer with blocking_read (cl_helper.py:262-302). */
int  adhip_read(adhip_ctx* ctx, uint64_t src_off, void* host, size_t bytes);
/* Staged host -> device copies on a transfer stream, overlapped with the
 * compute stream.  A staging set (tag 0..3) is opened, filled with copies
 * (each host buffer is copied to pinned memory before the call returns),
 * then closed: the compute stream waits for the set's copies before its
 * next work.  stage_release marks, on the compute stream, the point after
 * which the set's device data may be overwritten by the set's next round;
 * stage_begin makes the transfer stream wait for it.  This is how a Feeder
 * inside a replayed loop writes the next iteration's data while the current
 * one computes.  Replaces clEnqueueWriteBuffer (cl_helper.py:304-332) for
 * Feeders in loops. */
int  adhip_stage_begin(adhip_ctx* ctx, int tag);
int  adhip_stage_write(adhip_ctx* ctx, int tag, uint64_t dst_off, const void* host, size_t bytes);
int  adhip_stage_end(adhip_ctx* ctx, int tag);
int  adhip_stage_release(adhip_ctx* ctx, int tag);

/* Device -> host copies on the transfer stream into pinned memory, for
 * Receivers inside a replayed loop.  A fetch set (0..1) is reserved once
 * (pinned capacity), then per round: begin (the copies start after all
 * work queued on the compute stream so far), copy (returns where in the
 * set's pinned memory the bytes will land), end, and take (waits for the
 * set's copies on its first call, then copies into the caller's buffer).
 * A set must be taken before it begins again.  Replaces the blocking
 * clEnqueueReadBuffer of read_buffers (cl_helper.py:262-302) and the
 * unfinished read_buffers_async (cl_helper.py:176-260) for in-loop
 * Receivers. */
int  adhip_fetch_reserve(adhip_ctx* ctx, int set, size_t bytes);
int  adhip_fetch_begin(adhip_ctx* ctx, int set);
int  adhip_fetch_copy(adhip_ctx* ctx, int set, uint64_t src_off, size_t bytes, size_t* host_off);
int  adhip_fetch_end(adhip_ctx* ctx, int set);
int  adhip_fetch_take(adhip_ctx* ctx, int set, size_t host_off, void* dst, size_t bytes);

/* Stream-ordered device -> device copy inside the arena (capturable). */
int  adhip_copy(adhip_ctx* ctx, uint64_t dst_off, uint64_t src_off, size_t bytes);

/* hipRTC compile of a kernel module for the context's device (gfx950).
 * Thread-safe and context-free so callers may compile in parallel.  The
 * code object is returned in a malloc'd buffer (free with adhip_free).
 * Replaces clCreateProgramWithSource + clBuildProgram
 * (cl_helper.py:357-406). */
int  adhip_compile(const char* src, const char* options, void** code, size_t* code_size,
                   char* log, size_t log_cap);
void adhip_free(void* p);
/* Load a code object; look up kernels by name.  Replaces clCreateKernel
 * (cl_helper.py:388-400). */
int  adhip_module_load(adhip_ctx* ctx, const void* code, size_t code_size, adhip_module** out);
int  adhip_module_function(adhip_module* mod, const char* name, void** fn);

/* Launch `fn` with a packed argument buffer (every argument one 8-byte
 * slot: device pointers and int64 values).  Replaces clSetKernelArg +
 * clEnqueueNDRangeKernel (cl_helper.py:408-455). */
int  adhip_launch(adhip_ctx* ctx, void* fn, const uint32_t grid[3], const uint32_t block[3],
                  uint32_t shared_bytes, const uint64_t* args, size_t nargs);

/* Parallel launch lanes: `streams` compute streams in all (stream 0 is the
 * context stream; the others are created at default priority) and a pool of
 * `events` events.  launch_on / record_on / wait_on put a launch, an event
 * record or an event wait on a lane, so a captured graph gets parallel
 * branches with edges only where launches touch overlapping memory.  The
 * reference enqueues every command on one in-order queue
 * (cl_helper.py:128-139). */
int  adhip_lanes_reserve(adhip_ctx* ctx, int streams, int events);
int  adhip_launch_on(adhip_ctx* ctx, int stream, void* fn, const uint32_t grid[3], const uint32_t block[3],
                     uint32_t shared_bytes, const uint64_t* args, size_t nargs);
int  adhip_record_on(adhip_ctx* ctx, int stream, int event);
int  adhip_wait_on(adhip_ctx* ctx, int stream, int event);

/* Record the context stream's work between begin and end as a HIP graph,
 * then replay it.  The reference replays a loop body by re-enqueueing
 * every command from Python (device.py:121-129). */
int  adhip_graph_begin(adhip_ctx* ctx);
int  adhip_graph_end(adhip_ctx* ctx, adhip_graph** out);
/* End a capture whose work formed a chain of n_nodes graph nodes (kernel
 * launches and copies, in capture order) and replace the chain's edges by
 * the given dependencies before instantiating: node i follows the nodes
 * deps[dep_offsets[i] .. dep_offsets[i+1]) (earlier nodes only), so
 * independent launches of a loop body may run concurrently on replay.  The
 * reference replays a loop body command by command on one in-order queue
 * (device.py:114-124); the dependencies given must order every pair of
 * nodes touching overlapping memory, one of them writing. */
int  adhip_graph_end_dag(adhip_ctx* ctx, int32_t n_nodes, const int32_t* dep_offsets, const int32_t* deps,
                         adhip_graph** out);
int  adhip_graph_launch(adhip_ctx* ctx, adhip_graph* g);
void adhip_graph_destroy(adhip_graph* g);

/* Wait for all queued work.  Replaces clFinish (cl_helper.py:457-458). */
int  adhip_sync(adhip_ctx* ctx);

/* Column reduction of a row-major [rows, cols] fp32 matrix on device
 * memory: out[c] = SUM (op 0) or MAX (op 1) over r of x[r * cols + c],
 * enqueued on the context's stream.  The rows are split into chunks over
 * blocks; chunk results go to scratch the context allocates on first need
 * and keeps, and an ordered pass combines them.  Replaces the reduce
 * kernel (kernels/reduce.py:8-66) for a column reduction such as the
 * gamma/beta and bias gradients (graph/data/broadcast.py:18-21), with every
 * row combined (the reference's work-group tree reaches every element for
 * power-of-two row counts, reduce.py:38-43).  rows >= 1 when cols >= 1. */
int  adhip_reduce_cols(adhip_ctx* ctx, const float* x, float* out, uint32_t rows, uint32_t cols, int op);
/* adhip_reduce_cols without any allocation: the chunk results go to a
 * static device array of ADHIP_REDUCE_COLS_SCRATCH_FLOATS floats (one per
 * device, its address looked up once per device when a context is created)
 * instead of context-owned scratch.  No counterpart in the reference: for
 * callers that cannot allocate (code under HIP graph capture, serving loops
 * that forbid hipMalloc).  Same kernels and results as adhip_reduce_cols;
 * fails with ADHIP_E_ARG when chunks x cols exceed the array (the chunk
 * count follows the rows, at most 128; see the column reduction source).
 * Every call on one GPU shares that GPU's array: calls that overlap on one
 * GPU (other streams, contexts or threads) race. */
int  adhip_reduce_cols_noalloc(adhip_ctx* ctx, const float* x, float* out, uint32_t rows, uint32_t cols, int op);

/* Stream events for timing (milliseconds between two recorded events). */
int  adhip_event_record(adhip_ctx* ctx, int slot);
int  adhip_event_elapsed(adhip_ctx* ctx, int slot_a, int slot_b, float* ms);

#ifdef __cplusplus
}
#endif
#endif
