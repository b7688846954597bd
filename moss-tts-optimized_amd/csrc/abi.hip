// Library-level C-ABI helpers: version, error strings, device check.
#include "common.h"

MOSS_API int moss_abi_version(void) { return 1; }

MOSS_API const char* moss_error_string(int code) { return hipGetErrorString((hipError_t)code); }

// 0 when the current device is a gfx950 (MI350/MI355), hipErrorNoBinaryForGpu otherwise.
MOSS_API int moss_check_device(char* arch_out, int arch_len) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return (int)e;
    hipDeviceProp_t prop;
    e = hipGetDeviceProperties(&prop, dev);
    if (e != hipSuccess) return (int)e;
    if (arch_out && arch_len > 0) {
        int i = 0;
        for (; i < arch_len - 1 && prop.gcnArchName[i]; ++i) arch_out[i] = prop.gcnArchName[i];
        arch_out[i] = 0;
    }
    const char* want = "gfx950";
    for (int i = 0; want[i]; ++i)
        if (prop.gcnArchName[i] != want[i]) return (int)hipErrorNoBinaryForGpu;
    return 0;
}
