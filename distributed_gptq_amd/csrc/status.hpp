// Status plumbing of the C ABI (no HIP dependency): the thread-local message
// behind gptq_last_error() and the argument-check macro of the entry points.
#pragma once

#include "../../include/gptq_hip.h"

namespace gptq {

void set_error(const char* fmt, ...);
void clear_error();

}  // namespace gptq

#define GPTQ_REQUIRE(cond, code, ...)   \
  do {                                  \
    if (!(cond)) {                      \
      ::gptq::set_error(__VA_ARGS__);   \
      return (code);                    \
    }                                   \
  } while (0)
