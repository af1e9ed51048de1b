// Engine functions used by the model's allocation-free forward
// (dinov3_forward_noalloc); not part of the C ABI.
#pragma once
#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

#include "../../include/dinov3_engine.h"

namespace dhx {

// Adds a buffer slot that the engine does not own (never freed by it) over
// device memory at `ptr` of `bytes`; launches name it by the returned index
// like any allocated buffer. No allocation.
uint32_t engine_external(dhx_engine* e, void* ptr, uint64_t bytes);
// Points an external slot at other memory (another call's input or output).
void engine_rebind(dhx_engine* e, uint32_t buffer, void* ptr, uint64_t bytes);
// Validates every launch (bindings against the shapes their scalars imply),
// then queues them in order on `stream` with no graph; a launch failure
// poisons the engine as any failed HIP call does. Throws dhx::Error.
void engine_queue(dhx_engine* e, const dhx_launch* launches, size_t n, hipStream_t stream);
// The pipelined transfers of dhx_copy_in / dhx_copy_out_finish with the host
// copies left to the caller (the model's copier thread; none of these is
// called from it): the pinned staging buffers of a slot and their sizes;
// waiting until the slot's previous upload has left its input staging
// buffer; queueing the upload of n bytes of that buffer into dst (after the
// graph that last read dst for the slot); waiting until the slot's readback
// has landed in its output staging buffer.
void* engine_staging_in(dhx_engine* e, uint32_t slot);
void* engine_staging_out(dhx_engine* e, uint32_t slot);
uint64_t engine_staging_in_bytes(const dhx_engine* e);
uint64_t engine_staging_out_bytes(const dhx_engine* e);
void engine_wait_upload(dhx_engine* e, uint32_t slot);
void engine_upload(dhx_engine* e, dhx_region dst, uint64_t n, uint32_t slot);
void engine_wait_readback(dhx_engine* e, uint32_t slot);
// The engine's own stream and device.
hipStream_t engine_stream(const dhx_engine* e);
int engine_device(const dhx_engine* e);
// hip_check for callers outside the engine: poisons it on failure.
void engine_check(dhx_engine* e, hipError_t err, const char* what);
void engine_ensure_usable(const dhx_engine* e);

}  // namespace dhx
