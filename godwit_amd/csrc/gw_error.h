// gw_error.h — the library's error record: every C-ABI entry point returns a
// gw_status and leaves a message for gw_last_error() (thread-local).
#pragma once

namespace gw {
// Records the formatted message and returns `code`.
int set_error(int code, const char *fmt, ...) __attribute__((format(printf, 2, 3)));
}  // namespace gw
