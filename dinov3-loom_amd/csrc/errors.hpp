// Error type and the per-thread "last error" used before a handle exists.
#pragma once
#include <stdexcept>
#include <string>

namespace dhx {

struct Error : std::runtime_error {
    using std::runtime_error::runtime_error;
};

void set_global_error(const std::string& message);
const char* global_error();

}  // namespace dhx
