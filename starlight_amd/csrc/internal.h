// Library-internal entry points shared by the device and the engine (not
// part of the C ABI).
#ifndef STARLIGHT_INTERNAL_H
#define STARLIGHT_INTERNAL_H

#include "starlight_hip.h"

// Records `message` as the device's last error (status Execution), so a
// failing engine call is reported through sl_hip_last_error like a device
// call; returns SL_ERR_EXECUTION.
sl_status slhip_fail_execution(sl_hip_device* device, const char* message);

#endif
