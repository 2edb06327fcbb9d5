// rhizome_error.hpp -- the exception type of the C++ host layer
// (rhizome_delta.hpp, rhizome_plan.hpp, rhizome_exec.hpp).  It carries an
// rhz_status of include/rhizome_gdr.h: RHZ_ERR_INVALID_ARG for a shape or
// graph error (the reference's Error::Shape, crates/core/src/error.rs),
// RHZ_ERR_UNSUPPORTED for an (op, dtype, shape) the library does not run,
// RHZ_ERR_HIP for a failed HIP call.
#pragma once

#include <cstdint>
#include <stdexcept>
#include <string>

namespace rhizome {

class Error : public std::runtime_error {
public:
    Error(int32_t status, const std::string& what) : std::runtime_error(what), status_(status) {}
    int32_t status() const { return status_; }

private:
    int32_t status_;
};

namespace ops {
using rhizome::Error;
}  // namespace ops

}  // namespace rhizome
