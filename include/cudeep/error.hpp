// Error convention of the C++ host API: failures throw std::runtime_error,
// as the reference's CUDEEP_CHECK_CUDA / CUDEEP_ASSERT do
// (include/cudeep/error.cuh:11-40).  C-ABI status codes from
// libcudeep_amd.so are turned into exceptions carrying cdx_last_error().
#pragma once

#include <stdexcept>
#include <string>
#include <hip/hip_runtime_api.h>

#include "../cudeep_amd.h"

namespace cudeep {

inline void throw_hip(hipError_t e, const char* what, const char* file, int line) {
    throw std::runtime_error(std::string("HIP error: ") + hipGetErrorString(e) + " in " + what +
                             " at " + file + ":" + std::to_string(line));
}

inline void throw_cdx(int code, const char* what) {
    throw std::runtime_error(std::string(what) + " failed (status " + std::to_string(code) +
                             "): " + cdx_last_error());
}

}  // namespace cudeep

#define CUDEEP_CHECK_HIP(call)                                                   \
    do {                                                                         \
        hipError_t _e = (call);                                                  \
        if (_e != hipSuccess) ::cudeep::throw_hip(_e, #call, __FILE__, __LINE__); \
    } while (0)

#define CUDEEP_CHECK_CDX(call)                            \
    do {                                                  \
        int _s = (call);                                  \
        if (_s != CDX_OK) ::cudeep::throw_cdx(_s, #call); \
    } while (0)

#define CUDEEP_ASSERT(cond, msg)                                              \
    do {                                                                      \
        if (!(cond)) throw std::runtime_error(std::string("Assertion failed: ") + (msg)); \
    } while (0)
