// Helpers shared by the host-side translation units of the library (not part
// of the C ABI).
#pragma once
#include <string>

namespace lpi {

// Set this thread's lp_last_error() text and return `code`.
int set_error(int code, const std::string& msg);

}  // namespace lpi
