// Model/ModelError.h:16-20 — a user-facing shape or capacity error, thrown
// before anything is recorded.
#pragma once

#include <stdexcept>
#include <string>

namespace WSP
{
struct ModelError : std::runtime_error
{
    using std::runtime_error::runtime_error;
};
} // namespace WSP
