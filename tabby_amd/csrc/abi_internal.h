// Helpers shared by the library's translation units (not part of the C ABI): the calling
// thread's last-error message behind tabby_last_error(), and a HIP status check.
#pragma once

#include <hip/hip_runtime.h>

#include <string>

#include "tabby_sampler.h"

namespace tabby {

// Records `msg` as the calling thread's last error and returns `status`.
int record_failure(int status, const std::string &msg);

inline int record_hip_failure(hipError_t e, const char *what) {
  return record_failure(TABBY_EHIP, std::string(what) + ": " + hipGetErrorString(e));
}

// The device's compute-unit count (cached per device).
int device_cus(int device, int *cus);

// What the library's other kernels may use of a sampler handle: its device, its limits, and
// its candidate region as scratch (rows_max * vocab_max composites of 8 bytes). The scratch
// is shared with the sampling kernels; calls on one handle are stream-ordered and must not
// overlap, as for every entry point that takes a handle.
struct HandleView {
  int device;
  int cus;
  int32_t vocab_max, rows_max, k_max;
  void *scratch;
  size_t scratch_bytes;
};
int handle_view(const tabby_sampler *h, HandleView *out);

// The int4 lm_head's shape rules (hidden and block_size multiples of 32, block_size dividing
// hidden); TABBY_EINVAL with a message otherwise.
int check_q4_shape(int32_t vocab, int32_t hidden, int32_t block);

}  // namespace tabby

#define TABBY_HIP_CHECK(expr)                                            \
  do {                                                                   \
    hipError_t e_ = (expr);                                              \
    if (e_ != hipSuccess) return ::tabby::record_hip_failure(e_, #expr); \
  } while (0)
