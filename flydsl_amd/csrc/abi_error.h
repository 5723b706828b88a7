// Error reporting shared by the library's translation units: fail() formats the message that
// flygemm_last_error() returns on the calling thread and passes the error code through.
#pragma once

namespace flygemm {
__attribute__((visibility("hidden"))) int fail(int code, const char* fmt, ...)
    __attribute__((format(printf, 2, 3)));
}  // namespace flygemm
