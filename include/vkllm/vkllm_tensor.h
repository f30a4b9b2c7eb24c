/* 4-D tensors in HBM. Replaces src/core/vkllm_tensor.h:19-65.
 * Same field names and meaning as the reference: shapes [N,C,H,W], strides in BYTES with W innermost and no
 * padding, `bytes` the allocation size, `data.host`/`data.mapped`/`data.is_ref`, op/srcs/params for graph
 * nodes. `data.dev` is the device address that replaces the reference's VkBuffer. */
#ifndef VKLLM_TENSOR_H
#define VKLLM_TENSOR_H
#include <stdbool.h>
#include <stddef.h>
#include <stdint.h>
#include "vkllm_common.h"
#include "vkllm_dtypes.h"
#include "vkllm_ops.h"
#ifdef __cplusplus
extern "C" {
#endif

struct vkllm_context;
struct vkllm_pipeline;
struct vkllm_gpu_device;

struct vkllm_tensor
{
    const char name[128];
    vkllm_dtype_t dtype;
    uint32_t shapes[4];
    uint32_t strides[4];
    uint32_t bytes;

    struct vkllm_gpu_device *device;
    struct
    {
        void *dev;     /* HBM address of element [0,0,0,0]; NULL until first needed for op outputs */
        void *host;    /* pinned host mirror of a mapped tensor, else NULL */
        bool mapped;   /* has a host mirror (the reference's host-visible mapped buffer) */
        bool is_ref;   /* view: memory is srcs[0]'s, never freed here */
        bool borrowed; /* memory owned elsewhere (model weight slab), never freed here */
        bool valid;    /* device contents have been written (upload or op) */
        bool host_current; /* the host mirror holds the current contents (a fused step's arg-max output),
                              so invalid_cache and download read it without a device copy */
    } data;

    uint32_t access_flags;   /* kept for source compatibility; unused */
    uint32_t pipeline_stage; /* kept for source compatibility; unused */

    vkllm_op_t op;
    struct vkllm_pipeline *pipeline;
    struct vkllm_tensor *srcs[VKLLM_MAX_SRCS];
    uint8_t params[];
};

/* src/core/vkllm_tensor.c:66-145: zero shapes -> VKLLM_ERR_ARGS; params are copied into the tensor; mapped
 * tensors get a pinned host mirror. Device memory of op outputs is allocated on first use. */
extern vkllm_err_t vkllm_tensor_new(struct vkllm_context *context, const char *name, const uint32_t *shapes,
                                    vkllm_dtype_t dtype, vkllm_op_t op, struct vkllm_tensor **srcs,
                                    const uint32_t n_srcs, const void *params, size_t params_bytes, bool mapped,
                                    struct vkllm_tensor **p);
/* src/core/vkllm_tensor.c:147-160 */
extern void vkllm_tensor_free(struct vkllm_context *context, struct vkllm_tensor *tensor);
/* mapped tensors only (VKLLM_ERR_ARGS otherwise): device -> host mirror; src/core/vkllm_tensor.c:179-194 */
extern vkllm_err_t vkllm_tensor_invalid_cache(struct vkllm_context *context, struct vkllm_tensor *tensor);
/* mapped tensors only: host mirror -> device; src/core/vkllm_tensor.c:162-177 */
extern vkllm_err_t vkllm_tensor_flush_cache(struct vkllm_context *context, struct vkllm_tensor *tensor);
/* src/core/vkllm_tensor.c:196-203 */
extern vkllm_err_t vkllm_tensor_new_staging(struct vkllm_context *context, struct vkllm_tensor *tensor,
                                            struct vkllm_tensor **staging);
/* src/core/vkllm_tensor.c:221-238: element count must match; strides recomputed */
extern vkllm_err_t vkllm_tensor_reshape(struct vkllm_context *context, struct vkllm_tensor *tensor,
                                        const uint32_t *shapes);
/* src/core/vkllm_tensor.c:240-259: new dim i takes old dim axis[i] (shape and stride) */
extern vkllm_err_t vkllm_tensor_permute(struct vkllm_context *context, struct vkllm_tensor *tensor,
                                        const uint32_t *axis);
/* src/core/vkllm_tensor.c:261-299: op REF view sharing the memory, srcs[0] = tensor, name "<name>_ref" */
extern vkllm_err_t vkllm_tensor_copy_ref(struct vkllm_context *context, struct vkllm_tensor *tensor,
                                         struct vkllm_tensor **p);
/* src/core/vkllm_tensor.c:301-320: ref view with shapes shrunk to `extents`, strides kept */
extern vkllm_err_t vkllm_tensor_slice0(struct vkllm_context *context, struct vkllm_tensor *tensor,
                                       uint32_t extents[4], struct vkllm_tensor **slice);
/* src/core/vkllm_tensor.c:322-335: "name<dtype>[n, c, h, w]" */
extern vkllm_err_t vkllm_tensor_s(struct vkllm_context *context, struct vkllm_tensor *tensor, char *buf,
                                  size_t len);

#ifdef __cplusplus
}
#endif
#endif
