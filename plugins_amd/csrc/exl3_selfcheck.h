// exl3_selfcheck.h -- the load-time self-check exl3_open runs
// (exl3_selfcheck.cpp).
#pragma once

#include <hip/hip_runtime.h>

#include "../../include/exl3_mi355x.h"

namespace exl3 {

// device -1 runs the host part only (SHA-256 and the golden planes' code
// digests); else `device` is current and the device part runs for codebook
// form `form` (CB_FORM_MUL1 or CB_FORM_MCG) on stream s: once per process,
// device and form, once it has passed.
exl3_verdict self_check(int device, int form, hipStream_t s);

}  // namespace exl3
