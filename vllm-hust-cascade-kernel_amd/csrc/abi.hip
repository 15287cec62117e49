// abi.hip - ABI helpers shared by all entry points of libcascade_hip.so.
#include "ck_common.h"

extern "C" const char *ck_error_string(int code) {
    switch (code) {
        case CK_OK: return "success";
        case CK_E_INVALID_ARG: return "invalid argument (size, stride or mode outside the supported domain)";
        case CK_E_NULL_PTR: return "a required pointer is NULL";
        case CK_E_WORKSPACE: return "workspace missing or smaller than the plan requires";
        case CK_E_UNSUPPORTED: return "shape not supported by the built kernels";
        case CK_E_SCRATCH_LIMIT:
            return "the call needs more workspace than the no-allocation entry point's device scratch holds";
        default: break;
    }
    if (code > 0) return hipGetErrorString(static_cast<hipError_t>(code));
    return "unknown error";
}
