// Status reporting shared by every source file, device or host only.
#pragma once

#include "../../include/webgllm_hip.h"

namespace wg {

// Records the message for wg_last_error() and returns `code`.
int fail(int code, const char *fmt, ...) __attribute__((format(printf, 2, 3)));

}  // namespace wg

#define WG_REQUIRE(cond, ...)                                                          \
  do {                                                                                 \
    if (!(cond)) return ::wg::fail(WG_ERR_INVALID, __VA_ARGS__);                       \
  } while (0)
