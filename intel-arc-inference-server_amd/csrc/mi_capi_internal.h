// mi_capi_internal.h - error plumbing shared by the C-ABI entry points.
#pragma once
#include <stdint.h>

#include "../../include/mi355x_decode.h"

// Records `msg` as the calling thread's last error and returns `code`.
int mi_fail(int code, const char* msg);
// Returns `e` (a hipError_t value); records `where` and the HIP error string when non-zero.
int mi_hip(int e, const char* where);
// Whether the engine was created with an MTP head (its descriptor's mtp); for the loader.
extern "C" bool mi_engine_has_mtp(const mi_engine* e);
// Whether the engine runs bf16 activations (its descriptor's act_bf16); for the loader.
extern "C" bool mi_engine_act_bf16(const mi_engine* e);
