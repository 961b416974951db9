// Launch checks of the C ABI (the last-error message itself is in status.cpp).
#include "common.hpp"

namespace gptq {

int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_error("%s: launch failed: %s", what, hipGetErrorString(e));
    return GPTQ_ERR_LAUNCH;
  }
  return GPTQ_OK;
}

}  // namespace gptq
