// Shared pieces of the C ABI translation units.
#pragma once

#include <string>

#include "../../include/sdxl_hip/attention.h"

// Records `message` as this thread's sdxl_last_error() and returns status.
sdxl_status sdxl_hip_fail(sdxl_status status, const std::string& message);

// CUs of the current device, cached per device (0 if unknown); thread-safe.
int sdxl_hip_compute_units();
