// Host-side helpers shared by the C-ABI implementation files (not part of the ABI).
#pragma once

#include <hip/hip_runtime_api.h>

#include <algorithm>
#include <string>

#include "dcn_internal.hpp"

namespace dcn {
namespace host {

inline dcn_status fail(dcn_context* ctx, dcn_status status, const std::string& message) {
    if (ctx) ctx->last_error = message;
    return status;
}

inline dcn_status hip_fail(dcn_context* ctx, hipError_t e, const char* what) {
    return fail(ctx, DCN_COMMAND_FAILED, std::string(what) + ": " + hipGetErrorString(e));
}

#define DCN_HIP(ctx, expr)                                        \
    do {                                                          \
        hipError_t e_ = (expr);                                   \
        if (e_ != hipSuccess) return ::dcn::host::hip_fail((ctx), e_, #expr); \
    } while (0)

// Makes ctx->device current for the duration of a call.
struct DeviceGuard {
    int previous = -1;
    explicit DeviceGuard(int device) {
        if (hipGetDevice(&previous) == hipSuccess && previous != device) {
            (void)hipSetDevice(device);
        } else {
            previous = -1;
        }
    }
    ~DeviceGuard() {
        if (previous >= 0) (void)hipSetDevice(previous);
    }
};

// Owning device buffer for the host-pointer entry points.
struct DevBuf {
    void* p = nullptr;
    ~DevBuf() {
        if (p) (void)hipFree(p);
    }
};

inline dcn_status check_count(dcn_context* ctx, const char* name, size_t actual, size_t expected) {
    // DeformConvCPU.require (DeformConv.swift:140-144)
    if (actual != expected)
        return fail(ctx, DCN_INVALID_ARRAY_COUNT,
                    std::string(name) + " has " + std::to_string(actual) +
                        " elements; expected " + std::to_string(expected));
    return DCN_OK;
}

template <typename T>
dcn_status upload(dcn_context* ctx, DevBuf& buf, const T* host, size_t count) {
    DCN_HIP(ctx, hipMalloc(&buf.p, std::max<size_t>(count, 1) * sizeof(T)));
    if (count) DCN_HIP(ctx, hipMemcpy(buf.p, host, count * sizeof(T), hipMemcpyHostToDevice));
    return DCN_OK;
}

#define DCN_TRY(expr)                      \
    do {                                   \
        dcn_status st_ = (expr);           \
        if (st_ != DCN_OK) return st_;     \
    } while (0)


}  // namespace host
}  // namespace dcn
