// Shared host-side helpers: error propagation from the HIP runtime to the C ABI.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <string>

#include "paged_infer_amd.h"

namespace pia {

struct Error {
  pia_status code;
  std::string msg;
};

void set_last_error(const std::string& msg);

[[noreturn]] inline void fail(pia_status code, const std::string& msg) { throw Error{code, msg}; }

}  // namespace pia

#define PIA_HIP(call)                                                                          \
  do {                                                                                         \
    hipError_t pia_e_ = (call);                                                                \
    if (pia_e_ != hipSuccess)                                                                  \
      ::pia::fail(pia_e_ == hipErrorOutOfMemory ? PIA_ERR_OOM : PIA_ERR_HIP,                   \
                  std::string(#call) + " failed: " + hipGetErrorString(pia_e_));               \
  } while (0)

#define PIA_REQUIRE(cond, msg)                                                                 \
  do {                                                                                         \
    if (!(cond)) ::pia::fail(PIA_ERR_INVALID, std::string(msg));                               \
  } while (0)

// Wrap a C ABI body: exceptions become status codes + pia_last_error().
#define PIA_API_BEGIN try {
#define PIA_API_END                                                                            \
  return PIA_OK;                                                                               \
  }                                                                                            \
  catch (const ::pia::Error& e) {                                                              \
    ::pia::set_last_error(e.msg);                                                              \
    return e.code;                                                                             \
  }                                                                                            \
  catch (const std::exception& e) {                                                            \
    ::pia::set_last_error(e.what());                                                           \
    return PIA_ERR_INVALID;                                                                    \
  }
