// Error reporting shared by the C-ABI entry points (see include/loopsgl_tok.h).
#pragma once

#include <hip/hip_runtime.h>

#include "../../include/loopsgl_tok.h"

namespace lsg {

// Record a printf-style message in the calling thread's error slot; returns code.
int set_error(int code, const char* fmt, ...);
void clear_error();
// Turn a pending HIP launch error into LSG_ERR_HIP (message names `what`).
int check_launch(const char* what);

}  // namespace lsg
