// The library's per-thread error string (mono_last_error), for entry points defined
// outside abi.cpp.
#pragma once

namespace mono {
// record `msg` for mono_last_error() and return `code`
int abi_fail(int code, const char* msg);
// clear the error string and return MONO_OK
int abi_ok();
}  // namespace mono
