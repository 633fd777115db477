// Library-wide entry points: version, status strings, last HIP error.
#include "mf_common.h"

namespace mf {

static thread_local int g_last_hip_error = 0;

void set_last_hip_error(int err) { g_last_hip_error = err; }

int check_launch() {
    hipError_t err = hipGetLastError();
    if (err != hipSuccess) {
        set_last_hip_error((int)err);
        return MF_ERR_HIP;
    }
    return MF_OK;
}

}  // namespace mf

extern "C" const char* mf_version(void) { return "memforge_hip 0.1.0 (gfx950)"; }

extern "C" int mf_last_hip_error(void) { return mf::g_last_hip_error; }

extern "C" const char* mf_status_string(int status) {
    switch (status) {
        case MF_OK: return "ok";
        case MF_ERR_ARG: return "invalid argument";
        case MF_ERR_UNSUPPORTED: return "unsupported head_dim/dtype combination";
        case MF_ERR_WORKSPACE: return "workspace too small";
        case MF_ERR_HIP: return "HIP launch failed";
        default: return "unknown status";
    }
}
