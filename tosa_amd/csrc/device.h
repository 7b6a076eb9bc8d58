// HIP runtime plumbing: one stream per host thread, a stream-ordered caching
// allocator, and a per-stream device error word through which kernels report
// the reference's REQUIRE failures (src/ops/quant.rs:17-32,
// src/ops/type_conv.rs:183-186) without a host round trip per operator.
#pragma once

#include <hip/hip_runtime_api.h>

#include <cstddef>
#include <cstdint>

#include "core.h"

namespace tosa {

void hip_check(hipError_t e, const char* what);

// Error bits a kernel ORs into the error word.
enum DeviceErrorBits : uint32_t {
    DERR_SCALE_PARAMS = 1u << 0,   // multiplier < 0 or shift outside [2, 62]
    DERR_SCALE_RANGE = 1u << 1,    // value outside [-2^(shift-1), 2^(shift-1))
    DERR_SCALE_RESULT = 1u << 2,   // scaled result outside int32
    DERR_RESCALE_I32 = 1u << 3,    // result + output_zp outside int32
};
std::string device_error_message(uint32_t bits);

struct Stream {
    hipStream_t s = nullptr;
    uint32_t* err = nullptr;       // device error word of this stream
    uint32_t* err_host = nullptr;  // pinned host word it is read back into
};

// The calling thread's stream (created on first use), or the stream the
// caller installed with set_thread_stream().
Stream& thread_stream();
void set_thread_stream(hipStream_t s);

// Stream-ordered caching allocator: blocks freed on a stream are reused only
// for work later in the same stream.
void* dev_alloc(size_t bytes, hipStream_t s);
void dev_free(void* p, size_t bytes, hipStream_t s);
size_t dev_cached_bytes();

// Pinned host staging for uploads: pinned_acquire returns a page-locked
// block of at least `bytes`; pinned_release hands it back once the work
// enqueued on `s` so far (the copy out of it) has run, without waiting.
void* pinned_acquire(size_t bytes);
void pinned_release(void* p, hipStream_t s);

// Reset / read the error word of a stream (read synchronises the stream).
void clear_error_word(Stream& st);
uint32_t read_error_word(Stream& st);
// The device error word of stream `s` (created on first use; the one that
// thread_stream() carries when `s` is the thread's stream).
uint32_t* stream_error_word(hipStream_t s);

int device_count();
bool device_available();

}  // namespace tosa
