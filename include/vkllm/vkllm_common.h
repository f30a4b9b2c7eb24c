/* Shared macros, limits and host fp16 helpers.
 * Replaces src/core/vkllm_common.h:13-186: the same macro names and meanings (early return on error codes,
 * VKLLM_ERR_ARGS on a failed argument check), VKLLM_MAX_SRCS = 4, and the same host fp16 conversion behaviour
 * (truncating, subnormals flushed) the reference's tests use to build inputs. */
#ifndef VKLLM_COMMON_H
#define VKLLM_COMMON_H
#include <stddef.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include "vkllm_errors.h"
#ifdef __cplusplus
extern "C" {
#endif

#define VKLLM_MAX_PHY_DEVS 16
#define VKLLM_MAX_SRCS 4

/* logging: stderr, "[vkllm] LEVEL file:line: message" */
extern void vkllm_log(int level, const char *file, int line, const char *fmt, ...);
#define VKLLM_LOG_INFO 0
#define VKLLM_LOG_ERROR 1
#define log_info(...) vkllm_log(VKLLM_LOG_INFO, __FILE__, __LINE__, __VA_ARGS__)
#define log_error(...) vkllm_log(VKLLM_LOG_ERROR, __FILE__, __LINE__, __VA_ARGS__)

#define _NEW_AND_CHECK(_p, _type)                                                                                  \
    do                                                                                                             \
    {                                                                                                              \
        (_p) = (_type *)calloc(1, sizeof(_type));                                                                  \
        if (!(_p))                                                                                                 \
            return VKLLM_ERR_ALLOC;                                                                                \
    } while (0)

#define _NEW_N_AND_CHECK(_p, _type, _n)                                                                            \
    do                                                                                                             \
    {                                                                                                              \
        (_p) = (_type *)malloc(sizeof(_type) * (size_t)(_n));                                                      \
        if (!(_p))                                                                                                 \
            return VKLLM_ERR_ALLOC;                                                                                \
    } while (0)

#define _CHECK(_fn)                                                                                                \
    do                                                                                                             \
    {                                                                                                              \
        vkllm_err_t _vk_rc = (_fn);                                                                                \
        if (_vk_rc != VKLLM_ERR_OK)                                                                                \
            return _vk_rc;                                                                                         \
    } while (0)

#define _CHECK_JUMP(_fn, _ret, _label)                                                                             \
    do                                                                                                             \
    {                                                                                                              \
        (_ret) = (_fn);                                                                                            \
        if ((_ret) != VKLLM_ERR_OK)                                                                                \
            goto _label;                                                                                           \
    } while (0)

#define _CHECK_ARGS(_cond)                                                                                         \
    do                                                                                                             \
    {                                                                                                              \
        if (!(_cond))                                                                                              \
        {                                                                                                          \
            log_error("argument check failed: %s", #_cond);                                                        \
            return VKLLM_ERR_ARGS;                                                                                 \
        }                                                                                                          \
    } while (0)

#define BOOL_S(_c) ((_c) ? "true" : "false")
#define _MUL4(_v) ((_v)[0] * (_v)[1] * (_v)[2] * (_v)[3])
#define _ASSIGN4(_l, _r)                                                                                           \
    do                                                                                                             \
    {                                                                                                              \
        (_l)[0] = (_r)[0];                                                                                         \
        (_l)[1] = (_r)[1];                                                                                         \
        (_l)[2] = (_r)[2];                                                                                         \
        (_l)[3] = (_r)[3];                                                                                         \
    } while (0)
#define _DIV4_S(_v, _den, _out)                                                                                    \
    do                                                                                                             \
    {                                                                                                              \
        (_out)[0] = (_v)[0] / (_den);                                                                              \
        (_out)[1] = (_v)[1] / (_den);                                                                              \
        (_out)[2] = (_v)[2] / (_den);                                                                              \
        (_out)[3] = (_v)[3] / (_den);                                                                              \
    } while (0)
#define _ARRAY_SIZE(_a) (sizeof(_a) / sizeof((_a)[0]))
#define __UNUSED(_x) ((void)(_x))

/* 16-bit float storage word */
typedef struct
{
    uint16_t bits;
} vkllm_fp16_pack;

/* fp16 -> fp32 by field re-biasing; subnormal inputs become zero-exponent fp32 values as in the reference */
static inline float vkllm_fp16_to_fp32(vkllm_fp16_pack h)
{
    uint32_t sign = (uint32_t)(h.bits >> 15) & 1u, exp = (uint32_t)(h.bits >> 10) & 31u, frac = h.bits & 1023u;
    uint32_t out;
    if (exp == 31u)
        out = (sign << 31) | (255u << 23) | (frac ? 1u : 0u);
    else if (exp == 0u)
        out = (sign << 31) | (frac << 13);
    else
        out = (sign << 31) | ((exp + 112u) << 23) | (frac << 13);
    float f;
    memcpy(&f, &out, sizeof(f));
    return f;
}

/* fp32 -> fp16 by truncating the mantissa and clamping the exponent (not round-to-nearest) */
static inline vkllm_fp16_pack vkllm_fp32_to_fp16(float f)
{
    uint32_t x;
    memcpy(&x, &f, sizeof(x));
    uint32_t sign = x >> 31, exp = (x >> 23) & 255u, frac = x & 0x7fffffu;
    vkllm_fp16_pack h;
    if (exp == 255u && frac)
    {
        h.bits = (uint16_t)((sign << 15) | (31u << 10) | 1u);
        return h;
    }
    int e = (int)exp - 127;
    uint32_t he = e < -14 ? 0u : e > 15 ? 31u : (uint32_t)(e + 15);
    h.bits = (uint16_t)((sign << 15) | (he << 10) | (frac >> 13));
    return h;
}

#ifdef __cplusplus
}
#endif
#endif
