/* iris_internal.h - declarations shared by the HIP layer's translation units. */
#pragma once
#include "iris_dev.h"
#include "../../include/iris_hip.h"

hipStream_t iris_stream(void);
int iris_set_error(const char *fmt, ...);
int iris_check(hipError_t e, const char *what);
int iris_launch_check(const char *what);
