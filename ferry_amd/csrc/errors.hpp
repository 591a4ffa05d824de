// errors.hpp -- the library's last-error text, shared by every source file.
#pragma once

#include <string>

namespace ferry_amd {
// Record `msg` as this thread's ferry_last_error() text and return `code`.
int report(int code, const std::string& msg);
}  // namespace ferry_amd
