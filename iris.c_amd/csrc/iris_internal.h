/* iris_internal.h - declarations shared by the HIP layer's translation units. */
#pragma once
#include "iris_dev.h"
#include "../../include/iris_hip.h"

hipStream_t iris_stream(void);
int iris_cu_count(void);   /* compute units of the bound device (0 before init) */
int iris_set_error(const char *fmt, ...);
int iris_check(hipError_t e, const char *what);
int iris_launch_check(const char *what);

/* Per-launch timing for the library's profile (iris_hip_profile_enable):
 * while enabled and the stream is not being captured, each launch is
 * bracketed by two events on the library stream. begin returns the record
 * index, or -1 when nothing is recorded. */
int iris_prof_begin(const char *kernel, long long grid);
void iris_prof_end(int idx);

#define IRIS_LAUNCH(kernel, grid, block, smem, stream, ...)                                                   \
    do {                                                                                                      \
        const dim3 iris_grid_ = (grid);                                                                       \
        const int iris_prof_ = iris_prof_begin(#kernel, (long long)iris_grid_.x * iris_grid_.y * iris_grid_.z); \
        hipLaunchKernelGGL(kernel, iris_grid_, block, smem, stream, __VA_ARGS__);                            \
        iris_prof_end(iris_prof_);                                                                            \
    } while (0)
