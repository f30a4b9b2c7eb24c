/* Error codes. Replaces src/core/vkllm_errors.h:9-17 + src/core/vkllm_errors.inc:6-11 (same values: OK is 1). */
#ifndef VKLLM_ERRORS_H
#define VKLLM_ERRORS_H
#ifdef __cplusplus
extern "C" {
#endif

typedef enum
{
    VKLLM_ERR_START = 0,
    VKLLM_ERR_OK = 1,
    VKLLM_ERR_ALLOC = 2,
    VKLLM_ERR_VULKAN = 3, /* device-runtime failure; HIP errors are reported in this slot */
    VKLLM_ERR_DEV_NOT_FOUND = 4,
    VKLLM_ERR_PIPELINE_NOT_FOUND = 5,
    VKLLM_ERR_ARGS = 6,
} vkllm_err_t;

/* alias that names what the slot means on this backend */
#define VKLLM_ERR_DEVICE VKLLM_ERR_VULKAN

/* "VKLLM_ERR_OK" ... ; replaces src/core/vkllm_errors.h:17 */
extern const char *vkllm_err_s(vkllm_err_t err);

#ifdef __cplusplus
}
#endif
#endif
