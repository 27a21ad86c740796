// Internal interface between the host-only translation units (generate.cpp,
// gguf.cpp) and the library core (flare_hip.hip).  Not part of the C-ABI.
#pragma once

struct fl_ctx;

// Record `msg` as the error of ctx (or the global error when ctx is NULL,
// read by fl_last_error(NULL)) and return code.
int fl_host_fail(fl_ctx *ctx, int code, const char *msg);
