// Library-wide C ABI helpers (version, error strings).
#include "../../include/rwkv6_amd.h"

extern "C" {

int rwkv6_abi_version(void) { return RWKV6_ABI_VERSION; }

const char* rwkv6_strerror(int code) {
    switch (code) {
        case RWKV6_OK: return "ok";
        case RWKV6_ERR_INVALID_ARG: return "invalid argument (null pointer, size or dtype code)";
        case RWKV6_ERR_UNSUPPORTED: return "unsupported shape (head size must be 64)";
        case RWKV6_ERR_LAUNCH: return "kernel launch failed";
        case RWKV6_ERR_ALIGNMENT: return "tensor pointer not 16-byte aligned";
        default: return "unknown rwkv6 status code";
    }
}

}  // extern "C"
