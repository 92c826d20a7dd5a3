// Internal declarations shared by the library's translation units.
#pragma once
#include <hip/hip_runtime.h>
#include "../../include/krafla_hip.h"

hipStream_t kr_stream(void);
// records the first error (sticky) with a message
void kr_fail(ml_status st, const char *what, hipError_t e);
// records a launch error, if any
void kr_check_launch(const char *what);

// devices whose static scratch addresses the library keeps
constexpr int KR_MAX_DEVICES = 16;
// kr_attn.hip: takes this device's address of the attention scratch array
ml_status kr_attn_setup(int dev);
