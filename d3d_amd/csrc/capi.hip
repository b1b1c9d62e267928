// Library-wide entry points of libd3d_hip: status strings and version.
#include "../../include/d3d_hip.h"

#include <hip/hip_runtime.h>

extern "C" const char* d3d_status_string(int status) {
    switch (status) {
        case D3D_OK: return "ok";
        case D3D_E_SHAPE: return "invalid shape or size argument";
        case D3D_E_DTYPE: return "unsupported dtype";
        case D3D_E_WORKSPACE: return "workspace too small";
        case D3D_E_NULL: return "required pointer is NULL";
        case D3D_E_UNSUPPORTED: return "unsupported mode or parameter combination";
        case D3D_E_VALUE: return "scalar argument outside its domain";
        default:
            if (status > 0) return hipGetErrorString(static_cast<hipError_t>(status));
            return "unknown status";
    }
}

extern "C" int d3d_version(void) { return 100; }
