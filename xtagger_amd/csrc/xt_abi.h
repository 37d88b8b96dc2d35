// xt_abi.h - error convention of the C-ABI: every entry point returns 0, or -1 after printing
// "eva: <what>: <reason>" to stderr (the reference's EVA_CU convention, src/engine/eva.h:153-176). Every source that
// defines an exported entry point includes this file, and with it the public declarations of include/xtag_eva.h, so
// the compiler holds each definition to its declaration.
#pragma once
#include <hip/hip_runtime.h>
#include <stdio.h>

#include "xtag_eva.h"

static inline int xt_fail(const char *what, const char *why)
{
    fprintf(stderr, "eva: %s: %s\n", what, why);
    return -1;
}

static inline int xt_hip(hipError_t r, const char *what)
{
    if (r == hipSuccess) return 0;
    return xt_fail(what, hipGetErrorString(r));
}

static inline int xt_check(const char *what) { return xt_hip(hipGetLastError(), what); }

#define XT_HIP(call)                                 \
    do {                                             \
        if (xt_hip((call), #call)) return -1;        \
    } while (0)

// Compute units of the current device, read once per device and cached (0 if it cannot be read). Launchers that size
// a grid to what stays resident use it; the engines call it before their graph capture, so that no device query runs
// while a stream is being captured.
__attribute__((visibility("hidden"))) int xt_cu_count();
