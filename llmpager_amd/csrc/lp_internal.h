// Helpers shared by the host-side translation units of the library (not part
// of the C ABI).
#pragma once
#include <string>

struct lp_ctx;
struct lp_pack;

namespace lpi {

// Set this thread's lp_last_error() text and return `code`.
int set_error(int code, const std::string& msg);

// The device index a context was created on.
int ctx_device(const lp_ctx* c);

// Look up the allocation-free entry point's scratch array on `device` (the
// current device), once per device (lp_noalloc.hip).
int noalloc_setup(int device);

}  // namespace lpi
