// Internal host-side hooks shared by the runtime's source files: the
// thread-local last-error reporting behind ming_last_error and the
// context's device.
#pragma once

#include <string>

#include "../../include/ming_dit_amd.h"

namespace ming {
int rt_fail(int code, const std::string& why);
int rt_ok();
int rt_device(const ming_ctx* c);
// models hold their context like weights do: it refuses to go first
void rt_retain(ming_ctx* c);
void rt_release(ming_ctx* c);
}  // namespace ming
