// Shared C-ABI utilities: argument checks and error strings.
#include <hip/hip_runtime.h>

#include "fa_common.h"

namespace fa {
// Compute units of the current device, queried once per device (launch shapes).
int device_cus() {
    static int cached[64] = {0};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    if (cached[dev] == 0) {
        int n = 0;
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
        cached[dev] = n;
    }
    return cached[dev];
}

int check_tensor(const fa_tensor &t, bool required) {
    if (!t.ptr) return required ? FA_ERR_INVALID_ARG : FA_OK;
    if ((reinterpret_cast<uintptr_t>(t.ptr) & 15u) != 0) return FA_ERR_INVALID_ARG;
    if ((t.batch_stride & 7) || (t.row_stride & 7) || (t.head_stride & 7)) return FA_ERR_INVALID_ARG;
    return FA_OK;
}
}  // namespace fa

extern "C" const char *fa_error_string(int code) {
    switch (code) {
        case FA_OK:
            return "success";
        case FA_ERR_INVALID_ARG:
            return "fa_mi355x: invalid argument (shape, pointer, stride or alignment)";
        case FA_ERR_UNSUPPORTED:
            return "fa_mi355x: unsupported configuration (head_dim must be 64 or 128)";
        case FA_ERR_WORKSPACE:
            return "fa_mi355x: missing or too small workspace";
        case FA_ERR_SCRATCH:
            return "fa_mi355x: request needs more than the 16 MiB static scratch of fa_fwd_kvcache_noalloc "
                   "(fewer splits or a smaller batch, or fa_fwd_kvcache with a caller workspace)";
        default:
            return code > 0 ? hipGetErrorString(static_cast<hipError_t>(code)) : "fa_mi355x: unknown error";
    }
}

extern "C" int fa_abi_version(void) { return FA_ABI_VERSION; }
