// Shared host-side helpers: the host-only ones (errors, half conversion)
// plus HIP call checking.
#pragma once

#include <hip/hip_runtime.h>

#include "host_common.h"

#define OMG_HIP(call)                                                                   \
    do {                                                                                \
        hipError_t e_ = (call);                                                         \
        if (e_ != hipSuccess)                                                           \
            ::omg::fail(::omg::E_DEVICE, std::string(#call) + ": " + hipGetErrorString(e_)); \
    } while (0)
