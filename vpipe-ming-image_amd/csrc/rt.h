// Internal host-side hooks shared by the runtime's source files: the
// thread-local last-error reporting behind ming_last_error, the session log,
// device uploads and the context's device. Plain C++ (no HIP types), so the
// host-only sources include it too.
#pragma once

#include <cstddef>
#include <string>

#include "../../include/ming_dit_amd.h"

namespace ming {
int rt_fail(int code, const std::string& why);
int rt_ok();
int rt_device(const ming_ctx* c);
// models hold their context like weights do: it refuses to go first
void rt_retain(ming_ctx* c);
void rt_release(ming_ctx* c);
// the session log (ming_set_log_sink); level MING_LOG_WARN / MING_LOG_INFO
void rt_log(int level, const std::string& msg);
// a device copy of `bytes` host bytes on the context's device (NULL for 0)
int rt_upload(ming_ctx* c, const void* host, size_t bytes, void** dev);
void rt_free(ming_ctx* c, void* dev);
void rt_note_cap_hit(ming_ctx* c);
}  // namespace ming
