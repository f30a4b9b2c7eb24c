/* Kernel registry entries and per-kernel timing.
 * Replaces src/core/vkllm_pipeline.h:73-74 (vkllm_pipeline_query_exec_time) and the role of struct
 * vkllm_pipeline (which kernel a node runs). A pipeline names one HIP kernel family; when timing is enabled
 * (VKLLM_TIMING=1 or vkllm_hip_set_timing) each launch through it is bracketed with its own hipEvent pair;
 * the pairs are read at the next synchronisation point (vkllm_commands_wait_exec, vkllm_hip_synchronize, this
 * query), which keeps the last launch's duration like the reference's per-pipeline timestamp pair and also
 * the sum and count over all timed launches. */
#ifndef VKLLM_PIPELINE_H
#define VKLLM_PIPELINE_H
#include <stdint.h>
#include "vkllm_errors.h"
#ifdef __cplusplus
extern "C" {
#endif

struct vkllm_context;

struct vkllm_pipeline
{
    const char *name;
    int kernel_id;
    uint64_t last_ns;     /* duration of the last timed launch */
    uint64_t total_ns;    /* sum over timed launches */
    uint64_t launches;
    void *ev_begin, *ev_end; /* hipEvent_t of a launch being recorded (internal) */
    int pending;          /* event pairs were recorded but not yet read */
};

/* src/core/vkllm_pipeline.c:318-331: nanoseconds of the pipeline's last timed launch (waits for it) */
extern vkllm_err_t vkllm_pipeline_query_exec_time(struct vkllm_context *context, struct vkllm_pipeline *pipeline,
                                                  uint64_t *cost);

#ifdef __cplusplus
}
#endif
#endif
