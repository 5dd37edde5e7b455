// Host-side helpers shared by the library's translation units: the
// thread-local error message behind mtc_last_error() and launch checks.
#pragma once

#include <stddef.h>

namespace mtc {
namespace host {

// Records a formatted message for mtc_last_error() and returns `code`.
int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
// Clears the message and returns MTC_OK.
int ok();
// MTC_E_LAUNCH with the HIP error string if the last launch failed, else ok().
int check_launch(const char* what);
const char* last_error();
// LDS bytes one block may use on the current device.
size_t device_lds_limit();

}  // namespace host
}  // namespace mtc
