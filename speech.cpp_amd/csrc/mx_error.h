// The library's last-error message (mx_last_error), shared by its host-side sources.
#pragma once

namespace mx {
// Records `msg` as this thread's last error and returns `code`.
int set_error(int code, const char *msg);
}  // namespace mx
