// Error reporting shared by every source of the library (no HIP: the host
// parser builds without it): the thread's last error message and the typed
// status codes of llmhip.h.
#pragma once

#include <stdint.h>

#include "../../include/llmhip.h"

namespace llmhip {

// Records the thread's last error ("llm: ..."), returns code.
int set_error(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
void clear_error();
const char* last_error();

#define LLM_TRY(expr)     \
  do {                    \
    int r_ = (expr);      \
    if (r_ != 0) return r_; \
  } while (0)

}  // namespace llmhip
