/* Library context: one HIP device and its stream.
 * Replaces src/core/vkllm_context.h:19-112. The reference's table of ~186 Vulkan pipelines becomes the
 * kernel registry behind `pipelines`; `stats` keeps the reference's fields. */
#ifndef VKLLM_CONTEXT_H
#define VKLLM_CONTEXT_H
#include <stdint.h>
#include "vkllm_common.h"
#include "vkllm_errors.h"
#include "vkllm_ops.h"
#ifdef __cplusplus
extern "C" {
#endif

struct vkllm_gpu_device;     /* HIP device, stream, allocator (opaque) */
struct vkllm_pipeline_table; /* kernel registry (opaque) */
struct vkllm_hashmap;

struct vkllm_context
{
    const char *appname;
    struct vkllm_gpu_device *device;
    struct vkllm_pipeline_table *pipelines;
    struct
    {
        int tensor_alloc_counts;
        int tensor_free_counts;
        uint64_t op_time_costs[(int)VKLLM_OP_COUNTS];
        struct vkllm_hashmap *node_time_cost;
    } stats;
};

/* src/core/vkllm_context.c:8-27: `dev` indexes the HIP devices visible to the process;
 * VKLLM_ERR_DEV_NOT_FOUND when out of range. */
extern vkllm_err_t vkllm_context_new(uint32_t dev, struct vkllm_context **context);
/* src/core/vkllm_context.c:29-35 */
extern void vkllm_context_free(struct vkllm_context *context);

#ifdef __cplusplus
}
#endif
#endif
