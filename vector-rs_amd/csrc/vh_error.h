// vh_error.h -- the library's thread-local error state (host code, no HIP types), like the
// Result<_, CudaError> of each reference call (vector-cuda/src/error.rs:7-29).
#pragma once

#include <cstddef>
#include <string>

namespace vh {

// Records `msg` for vhip_last_error() and returns `code`.
int set_error(int code, const std::string &msg);
// Records an InsufficientDevices{requested, available} error.
void set_insufficient(size_t requested, size_t available);
// Records a DeviceNotFound{ordinal} error and returns its status.
int set_device_not_found(int ordinal, const std::string &msg);
void clear_error();

}  // namespace vh
