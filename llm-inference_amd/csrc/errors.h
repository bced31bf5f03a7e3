// Host-side error reporting shared by every translation unit of the library.
#pragma once

#include <hip/hip_runtime_api.h>

// Records or reports an error: prints to stderr and exits when the exit-on-error mode is on
// (the reference's behaviour, src/common.cuh:11-22), else keeps the message for
// llm_last_error(). Returns false so callers can write `if (!check(...)) return;`.
bool llm_fail(const char *fmt, ...) __attribute__((format(printf, 1, 2)));
bool llm_has_error();

#define HIP_OK(call)                                                                       \
    ([&]() -> bool {                                                                       \
        hipError_t err_ = (call);                                                          \
        if (err_ != hipSuccess)                                                            \
            return llm_fail("HIP error at %s:%d: %s\n  %s", __FILE__, __LINE__,            \
                            hipGetErrorString(err_), #call);                               \
        return true;                                                                       \
    }())

// Checks the launch of the kernel just issued (errors of the kernel itself show up at the
// next synchronisation).
#define LAUNCH_OK() HIP_OK(hipGetLastError())
