// lm_error.h -- the library's thread-local error message, shared by the host-only
// translation units (the message lm_last_error returns).
#pragma once

#include <string>

namespace lm {
// Stores `message` for lm_last_error and returns `code`.
int set_error(int code, const std::string& message);
}  // namespace lm
