/* Per-layer fp16 K/V caches [1, n_head, ctx, head_dim]. Replaces src/models/vkllm_kvcache.h:9-25. */
#ifndef VKLLM_KVCACHE_H
#define VKLLM_KVCACHE_H
#include <stdint.h>
#include "vkllm_errors.h"
#ifdef __cplusplus
extern "C" {
#endif

struct vkllm_array_tensor;
struct vkllm_tensor;
struct vkllm_context;

struct vkllm_kvcache
{
    struct vkllm_array_tensor *kcaches;
    struct vkllm_array_tensor *vcaches;
    uint32_t kcache_shape[4];
    uint32_t vcache_shape[4];
    uint32_t layer_counts;
    void *priv; /* views handed out by vkllm_kvcache_update, released with the cache */
};

/* src/models/vkllm_kvcache.c:12-63: caches are UPDATE_ROWS tensors, zero-filled */
extern vkllm_err_t vkllm_kvcache_new(struct vkllm_context *context, uint32_t kcache_shape[4],
                                     uint32_t vcache_shape[4], uint32_t layer_counts, struct vkllm_kvcache **kvcache);
/* src/models/vkllm_kvcache.c:65-102: wires *key / *value as the caches' sources at row `offset` and replaces
 * them with views [b, c, offset + rows, w] of the caches */
extern vkllm_err_t vkllm_kvcache_update(struct vkllm_context *context, struct vkllm_kvcache *kvcache,
                                        struct vkllm_tensor **key, struct vkllm_tensor **value, uint32_t layer,
                                        uint32_t offset);
extern void vkllm_kvcache_free(struct vkllm_context *context, struct vkllm_kvcache *kvcache);

#ifdef __cplusplus
}
#endif
#endif
