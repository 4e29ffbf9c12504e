// Library-level entry points of libpointops_hip.so.
#include <string.h>

#include "pointops_hip.h"

extern "C" {

int pointops_abi_version(void) { return 1; }

int pointops_device_supported(int device) {
    hipDeviceProp_t prop;
    if (hipGetDeviceProperties(&prop, device) != hipSuccess) return 0;
    return strncmp(prop.gcnArchName, "gfx950", 6) == 0 ? 1 : 0;
}

}  // extern "C"
