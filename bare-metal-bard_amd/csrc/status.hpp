// Launch-status bookkeeping shared by host-only and HIP translation units.
#pragma once

#include <hip/hip_runtime_api.h>

namespace bmb {

// Records a failed launch status for the calling host thread; the first
// failure since the last bmb_last_error() call is kept.
void note_launch_status(hipError_t e);

}  // namespace bmb
