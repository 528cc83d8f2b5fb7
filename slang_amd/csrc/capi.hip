// Host-side pieces of the C ABI shared by every entry point: error reporting and
// config validation. Kernels live in decode.hip, prefill.hip and kv_write.hip.
#include <stdarg.h>
#include <stdio.h>

#include "common.hpp"

namespace g4a {

static thread_local char g_last_error[512] = "";

void set_error(const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_last_error, sizeof g_last_error, fmt, ap);
    va_end(ap);
}

int hip_error(hipError_t e, const char* what) {
    set_error("%s: %s", what, hipGetErrorString(e));
    return G4A_EHIP;
}

bool check_cfg(const g4a_cfg* cfg, bool need_group_le8) {
    if (!cfg) {
        set_error("cfg is NULL");
        return false;
    }
    if (cfg->n_q_heads == 0 || cfg->n_kv_heads == 0 || cfg->n_q_heads % cfg->n_kv_heads) {
        set_error("n_q_heads (%u) must be a positive multiple of n_kv_heads (%u)", cfg->n_q_heads,
                  cfg->n_kv_heads);
        return false;
    }
    if (need_group_le8) {
        uint32_t g = cfg->n_q_heads / cfg->n_kv_heads;
        if (g != 1 && g != 2 && g != 4 && g != 8) {
            set_error("query heads per kv head must be 1, 2, 4 or 8 (got %u)", g);
            return false;
        }
    }
    if (!(cfg->eps >= 0.0f) || !(cfg->scale > 0.0f) || !(cfg->out_q >= 0.0f)) {
        set_error("eps/out_q must be >= 0 and scale > 0");
        return false;
    }
    return true;
}

}  // namespace g4a

extern "C" {

const char* g4a_strerror(int code) {
    switch (code) {
        case G4A_OK: return "ok";
        case G4A_EINVAL: return "invalid argument";
        case G4A_EUNSUPPORTED: return "unsupported shape";
        case G4A_EWORKSPACE: return "workspace too small";
        case G4A_EHIP: return "HIP error";
        default: return "unknown error";
    }
}

const char* g4a_last_error(void) { return g4a::g_last_error; }

int g4a_version(void) { return G4A_VERSION; }

}  // extern "C"
