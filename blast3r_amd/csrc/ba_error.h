// Error reporting for the C ABI: every entry point returns 0 on success and a
// nonzero code otherwise, with a thread-local message behind ba_last_error().
#pragma once
#include <hip/hip_runtime.h>
#include <string>

namespace ba {
void set_error(const std::string& msg);
void clear_error();
}  // namespace ba

#define BA_OK 0
#define BA_ERR_ARG 1
#define BA_ERR_HIP 2
#define BA_ERR_UNSUPPORTED 3

#define BA_REQUIRE(cond, msg)                                   \
    do {                                                        \
        if (!(cond)) { ::ba::set_error(msg); return BA_ERR_ARG; } \
    } while (0)

#define BA_HIP(call)                                                                   \
    do {                                                                               \
        hipError_t e_ = (call);                                                        \
        if (e_ != hipSuccess) {                                                        \
            ::ba::set_error(std::string(#call) + ": " + hipGetErrorString(e_));         \
            return BA_ERR_HIP;                                                         \
        }                                                                              \
    } while (0)

#define BA_LAUNCHED()                                                                  \
    do {                                                                               \
        hipError_t e_ = hipGetLastError();                                             \
        if (e_ != hipSuccess) {                                                        \
            ::ba::set_error(std::string("kernel launch: ") + hipGetErrorString(e_));    \
            return BA_ERR_HIP;                                                         \
        }                                                                              \
    } while (0)
