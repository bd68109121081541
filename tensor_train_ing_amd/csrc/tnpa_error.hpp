// The thread-local error message behind tnpa_last_error(), shared by every C-ABI translation unit of libtnpa.so.
#pragma once

namespace tnpa {
// Records a formatted message for tnpa_last_error() and returns code.
int set_error(int code, const char* fmt, ...);
// Clears the message and returns 0.
int clear_error();
}  // namespace tnpa
