// Host-side helpers shared by the entry points: error reporting, device facts.
#pragma once
#include <hip/hip_runtime.h>

#include "../../include/gstar_evict.h"

// Records `msg` as the calling thread's last error and returns `code`.
int gse_fail(int code, const char* msg);
// Turns a pending launch error into GSE_ELAUNCH with the HIP error text.
int gse_launch_check(const char* what);
// Compute units of the current device (cached per device; 256 if the query fails).
int gse_device_cus();
