// Internal interface between the translation units of libadhip.so (not
// exported): the context's stream, error reporting and device memory the
// context owns, for entry points defined outside adhip.cpp.
#ifndef ADHIP_INTERNAL_H
#define ADHIP_INTERNAL_H
#include <hip/hip_runtime.h>

#include "../../include/adhip.h"

namespace adhip_internal {
hipStream_t stream_of(adhip_ctx* ctx);
// Record the message on the context (thread-local when ctx is null) and
// return the code.
int fail_arg(adhip_ctx* ctx, const char* fmt, ...);
int fail_state(adhip_ctx* ctx, const char* fmt, ...);
int fail_hip(adhip_ctx* ctx, hipError_t e, const char* what);
// At least `bytes` of device memory owned by the context (hipMalloc on first
// need, reallocated larger when a call needs more, freed by adhip_destroy).
// Refused while the context's stream is being captured.
int workspace(adhip_ctx* ctx, size_t bytes, void** ptr);
// The context device's address of the column reduction's static scratch
// array (looked up in adhip_create), or null.
void* static_scratch(adhip_ctx* ctx);
// hipGetSymbolAddress of that array on the current device (defined beside it).
int scratch_symbol(int device, void** ptr);
}  // namespace adhip_internal

#endif
