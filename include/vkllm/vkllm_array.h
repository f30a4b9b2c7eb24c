/* Growable arrays used in public structs (graph node lists, token tables).
 * Replaces src/core/vkllm_array.h:17-85: VKLLM_DEF_ARRAY(name, type) defines struct vkllm_array_<name>
 * {alloc_n, used_n, data} with _new/_copy/_append/_free. */
#ifndef VKLLM_ARRAY_H
#define VKLLM_ARRAY_H
#include "vkllm_common.h"
#include "vkllm_dtypes.h"
#ifdef __cplusplus
extern "C" {
#endif

#define VKLLM_DEF_ARRAY(_name, _type)                                                                              \
    struct vkllm_array_##_name                                                                                     \
    {                                                                                                              \
        size_t alloc_n;                                                                                            \
        size_t used_n;                                                                                             \
        _type *data;                                                                                               \
    };                                                                                                             \
    static inline vkllm_err_t vkllm_array_##_name##_new(struct vkllm_array_##_name **arr, size_t init)             \
    {                                                                                                              \
        struct vkllm_array_##_name *a = (struct vkllm_array_##_name *)calloc(1, sizeof(*a));                       \
        if (!a)                                                                                                    \
            return VKLLM_ERR_ALLOC;                                                                                \
        a->alloc_n = init > 0 ? init : 1;                                                                          \
        a->data = (_type *)malloc(sizeof(_type) * a->alloc_n);                                                     \
        if (!a->data)                                                                                              \
        {                                                                                                          \
            free(a);                                                                                               \
            return VKLLM_ERR_ALLOC;                                                                                \
        }                                                                                                          \
        *arr = a;                                                                                                  \
        return VKLLM_ERR_OK;                                                                                       \
    }                                                                                                              \
    static inline vkllm_err_t vkllm_array_##_name##_append(struct vkllm_array_##_name *a, _type v)                 \
    {                                                                                                              \
        if (a->used_n == a->alloc_n)                                                                               \
        {                                                                                                          \
            size_t n = a->alloc_n * 2;                                                                             \
            _type *d = (_type *)realloc((void *)a->data, sizeof(_type) * n);                                       \
            if (!d)                                                                                                \
                return VKLLM_ERR_ALLOC;                                                                            \
            a->data = d;                                                                                           \
            a->alloc_n = n;                                                                                        \
        }                                                                                                          \
        a->data[a->used_n++] = v;                                                                                  \
        return VKLLM_ERR_OK;                                                                                       \
    }                                                                                                              \
    static inline vkllm_err_t vkllm_array_##_name##_copy(struct vkllm_array_##_name *src,                          \
                                                         struct vkllm_array_##_name **dst)                         \
    {                                                                                                              \
        vkllm_err_t rc = vkllm_array_##_name##_new(dst, src->alloc_n);                                             \
        if (rc != VKLLM_ERR_OK)                                                                                    \
            return rc;                                                                                             \
        memcpy((void *)(*dst)->data, (const void *)src->data, sizeof(_type) * src->used_n);                        \
        (*dst)->used_n = src->used_n;                                                                              \
        return VKLLM_ERR_OK;                                                                                       \
    }                                                                                                              \
    static inline void vkllm_array_##_name##_free(struct vkllm_array_##_name *a)                                   \
    {                                                                                                              \
        if (!a)                                                                                                    \
            return;                                                                                                \
        free((void *)a->data);                                                                                     \
        free(a);                                                                                                   \
    }

VKLLM_DEF_ARRAY(ptr, void *)
VKLLM_DEF_ARRAY(u8, uint8_t)
VKLLM_DEF_ARRAY(u32, uint32_t)
VKLLM_DEF_ARRAY(f32, float)
VKLLM_DEF_ARRAY(dtype, vkllm_dtype_t)

#ifdef __cplusplus
}
#endif
#endif
