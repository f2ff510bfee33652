// Host-only helpers shared by the library's C++ sources (no HIP types).
#pragma once

namespace gl3 {

// Records a formatted message for gl3_last_error() on this thread and returns code.
int host_fail(int code, const char *fmt, ...) __attribute__((format(printf, 2, 3)));

}  // namespace gl3
