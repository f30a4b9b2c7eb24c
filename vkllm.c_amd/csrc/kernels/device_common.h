// Device-side helpers shared by the gfx950 kernels: fp16 casts (round-to-nearest-even), strided element access,
// wave64 and workgroup reductions.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "kernels.h"

namespace vk
{

constexpr int kWave = 64;

// Raises a kernel's dynamic LDS limit above the default 64 KB on the current device. The attribute is per device,
// so `done` keeps one bit per device ordinal that has it (ordinals past 63 set it on every call).
inline hipError_t lds_attr_once(const void *fn, size_t bytes, uint64_t &done)
{
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess)
        return e;
    const uint64_t bit = dev >= 0 && dev < 64 ? 1ull << dev : 0;
    if (bit && (__atomic_load_n(&done, __ATOMIC_ACQUIRE) & bit))
        return hipSuccess;
    e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)bytes);
    if (e == hipSuccess && bit)
        __atomic_fetch_or(&done, bit, __ATOMIC_RELEASE);
    return e;
}

// Resident workgroups per CU of `fn` at `threads` threads and `lds` bytes of dynamic LDS on the current device, or -1
// when the query fails. `memo` keeps the last answer in one word (LDS bytes in bits 32-63, device in 24-31, a valid
// bit at 16, the count in 0-15), so callers on several threads or devices never pair a count with another size.
inline int occupancy_per_cu(const void *fn, int threads, size_t lds, uint64_t &memo)
{
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess)
        return -1;
    const uint64_t key = ((uint64_t)(uint32_t)lds << 32) | ((uint64_t)(dev & 0xff) << 24) | (1ull << 16);
    const uint64_t m = __atomic_load_n(&memo, __ATOMIC_ACQUIRE);
    if (lds <= 0xffffffffu && (m & ~0xffffull) == key)
        return (int)(m & 0xffff);
    int n = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, fn, threads, lds) != hipSuccess)
        return -1;
    if (lds <= 0xffffffffu && n >= 0 && n <= 0xffff)
        __atomic_store_n(&memo, key | (uint64_t)n, __ATOMIC_RELEASE);
    return n;
}

__device__ __forceinline__ float h2f(uint16_t h)
{
    _Float16 v;
    __builtin_memcpy(&v, &h, 2);
    return (float)v;
}

__device__ __forceinline__ uint16_t f2h(float f)
{
    // The empty asm pins f as a rounded fp32 register value. Without it the backend folds fp16(a * b) into one
    // v_fma_mixlo_f16 (exact product rounded once to fp16), which differs from rounding to fp32 and then to fp16.
    asm("" : "+v"(f));
    _Float16 v = (_Float16)f; // v_cvt_f16_f32, round-to-nearest-even
    uint16_t h;
    __builtin_memcpy(&h, &v, 2);
    return h;
}

__device__ __forceinline__ size_t voff(const TView &t, uint32_t b, uint32_t c, uint32_t h, uint32_t w)
{
    return (size_t)b * t.s[0] + (size_t)c * t.s[1] + (size_t)h * t.s[2] + (size_t)w * t.s[3];
}

__device__ __forceinline__ float ldf(const TView &t, size_t off)
{
    switch (t.dt)
    {
    case DT_F32:
        return ((const float *)t.p)[off];
    case DT_F16:
        return h2f(((const uint16_t *)t.p)[off]);
    case DT_U32:
        return (float)((const uint32_t *)t.p)[off];
    default:
        return (float)((const int8_t *)t.p)[off];
    }
}

__device__ __forceinline__ void stf(const TView &t, size_t off, float v)
{
    switch (t.dt)
    {
    case DT_F32:
        ((float *)t.p)[off] = v;
        break;
    case DT_F16:
        ((uint16_t *)t.p)[off] = f2h(v);
        break;
    case DT_U32:
        ((uint32_t *)t.p)[off] = (uint32_t)v;
        break;
    default:
        ((int8_t *)t.p)[off] = (int8_t)v;
        break;
    }
}

// index -> (b, c, h, w) of shape n
__device__ __forceinline__ void unflatten(uint64_t i, const uint32_t n[4], uint32_t &b, uint32_t &c, uint32_t &h,
                                          uint32_t &w)
{
    w = (uint32_t)(i % n[3]);
    i /= n[3];
    h = (uint32_t)(i % n[2]);
    i /= n[2];
    c = (uint32_t)(i % n[1]);
    b = (uint32_t)(i / n[1]);
}

__device__ __forceinline__ float wave_sum(float v)
{
#pragma unroll
    for (int o = 32; o > 0; o >>= 1)
        v += __shfl_xor(v, o, kWave);
    return v;
}

__device__ __forceinline__ float wave_max(float v)
{
#pragma unroll
    for (int o = 32; o > 0; o >>= 1)
        v = fmaxf(v, __shfl_xor(v, o, kWave));
    return v;
}

// Sum over the workgroup; `red` holds one float per wave. All threads get the result.
__device__ __forceinline__ float block_sum(float v, float *red)
{
    const int lane = threadIdx.x & (kWave - 1), wid = threadIdx.x / kWave, nw = (blockDim.x + kWave - 1) / kWave;
    v = wave_sum(v);
    __syncthreads();
    if (lane == 0)
        red[wid] = v;
    __syncthreads();
    float r = 0.f;
    for (int i = 0; i < nw; ++i)
        r += red[i];
    return r;
}

__device__ __forceinline__ float block_max(float v, float *red)
{
    const int lane = threadIdx.x & (kWave - 1), wid = threadIdx.x / kWave, nw = (blockDim.x + kWave - 1) / kWave;
    v = wave_max(v);
    __syncthreads();
    if (lane == 0)
        red[wid] = v;
    __syncthreads();
    float r = red[0];
    for (int i = 1; i < nw; ++i)
        r = fmaxf(r, red[i]);
    return r;
}

__device__ __forceinline__ float silu(float v)
{
    return v / (1.0f + expf(-v));
}

// Order of the reference's ARG_MAX (src/shaders/vkllm_arg_max.comp:40-97). There, lane l of 32 keeps the first
// maximum among elements i == l (mod 32) (strict '>'), then a strict-'>' tree over lane strides 16, 8, 4, 2, 1 keeps
// the lower lane on ties, so lane bit 0 decides first, then bit 1, and so on. Among equal maxima the winner is the
// index whose lane has the smallest 5-bit bit reversal, then the smallest index. As a comparison of (value, index)
// pairs that is a total order, so a reduction in any grouping returns the reference's answer.
__device__ __forceinline__ uint32_t lane_rank(uint32_t i)
{
    return __brev(i & 31u) >> 27;
}

// true when (v, i) comes before (w, k) in that order
__device__ __forceinline__ bool am_before(float v, uint32_t i, float w, uint32_t k)
{
    if (v != w)
        return v > w;
    const uint32_t ri = lane_rank(i), rk = lane_rank(k);
    return ri != rk ? ri < rk : i < k;
}

// ---- 16-byte vectors of fp16 pairs, dot products and DPP reductions ----
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float half_lo(uint32_t v)
{
    return h2f((uint16_t)(v & 0xffffu));
}
__device__ __forceinline__ float half_hi(uint32_t v)
{
    return h2f((uint16_t)(v >> 16));
}

// 8-element fp16 dot product accumulated in fp32 (fp16 -> fp32 widening FMAs, v_fma_mix_f32). The
// v_dot2_f32_f16 builtin gave wrong sums on gfx950 and is not used.
__device__ __forceinline__ float dot8(u32x4 w, u32x4 x, float acc)
{
#pragma unroll
    for (int i = 0; i < 4; ++i)
    {
        acc = fmaf(half_lo(w[i]), half_lo(x[i]), acc);
        acc = fmaf(half_hi(w[i]), half_hi(x[i]), acc);
    }
    return acc;
}
__device__ __forceinline__ uint32_t pack2(uint16_t lo, uint16_t hi)
{
    return (uint32_t)lo | ((uint32_t)hi << 16);
}

// fp16(fp16(up) * fp16(silu(gate))) as the reference's ffn_up_and_gate rounds it
__device__ __forceinline__ uint16_t swiglu_out(float up, float gate)
{
    return f2h(h2f(f2h(up)) * h2f(f2h(silu(gate))));
}

// Prompt-step activations of at most 128 rows (tokens) kept in the operand order of v_mfma_f32_32x32x16_f16's B
// matrix over 32-token blocks, so a wave reads one 16-K step of one token block as 1 KB contiguous: the 16-byte
// vector holding row t, columns 8 kv .. 8 kv + 7 of an [M <= 128, K] fp16 matrix is vector number
// (kv / 2 * 4 + t / 32) * 64 + (kv % 2) * 32 + t % 32. The matrix takes 128 * K halfs whatever M is.
__device__ __forceinline__ uint32_t xt_vec(uint32_t t, uint32_t kv)
{
    return ((kv / 2) * 4 + t / 32) * 64 + (kv % 2) * 32 + t % 32;
}

// normalises row `x` (D fp16) into `dst` (8 halfs per u32x4); all threads of the block take part. With
// xt_row >= 0, dst is a fragment-ordered activation matrix (xt_vec) and the row is its row xt_row.
__device__ __forceinline__ void rmsnorm_row_to(const uint16_t *x, const float *w, u32x4 *dst, uint32_t D, float eps,
                                               float *red, int xt_row = -1)
{
    const uint32_t nv = D / 8;
    const u32x4 *xv = (const u32x4 *)x;
    const float4 *wv = (const float4 *)w;
    if (nv <= blockDim.x)
    {
        // one vector per thread: the row and its weights are read once, before the reduction, and kept in
        // registers (the same sums in the same order as the loop below)
        const uint32_t i = threadIdx.x;
        u32x4 v = (u32x4){0, 0, 0, 0};
        float4 w0 = {0.f, 0.f, 0.f, 0.f}, w1 = w0;
        if (i < nv)
        {
            v = xv[i];
            w0 = wv[2 * i];
            w1 = wv[2 * i + 1];
        }
        float ss = 0.f;
#pragma unroll
        for (int k = 0; k < 4; ++k)
        {
            float a = half_lo(v[k]), b = half_hi(v[k]);
            ss += a * a;
            ss += b * b;
        }
        ss = block_sum(ss, red);
        const float alpha = 1.0f / sqrtf(ss / (float)D + eps);
        if (i < nv)
        {
            const float ws[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
            u32x4 o;
#pragma unroll
            for (int k = 0; k < 4; ++k)
            {
                float a = half_lo(v[k]), b = half_hi(v[k]);
                o[k] = pack2(f2h((a * ws[2 * k]) * alpha), f2h((b * ws[2 * k + 1]) * alpha));
            }
            dst[xt_row < 0 ? i : xt_vec((uint32_t)xt_row, i)] = o;
        }
        return;
    }
    float ss = 0.f;
    for (uint32_t i = threadIdx.x; i < nv; i += blockDim.x)
    {
        u32x4 v = xv[i];
#pragma unroll
        for (int k = 0; k < 4; ++k)
        {
            float a = half_lo(v[k]), b = half_hi(v[k]);
            ss += a * a;
            ss += b * b;
        }
    }
    ss = block_sum(ss, red);
    const float alpha = 1.0f / sqrtf(ss / (float)D + eps);
    for (uint32_t i = threadIdx.x; i < nv; i += blockDim.x)
    {
        u32x4 v = xv[i];
        float4 w0 = wv[2 * i], w1 = wv[2 * i + 1];
        float ws[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
        u32x4 o;
#pragma unroll
        for (int k = 0; k < 4; ++k)
        {
            float a = half_lo(v[k]), b = half_hi(v[k]);
            o[k] = pack2(f2h((a * ws[2 * k]) * alpha), f2h((b * ws[2 * k + 1]) * alpha));
        }
        dst[xt_row < 0 ? i : xt_vec((uint32_t)xt_row, i)] = o;
    }
}

// wave64 sum with DPP: row reductions (quad_perm, half-row and row mirrors), then row_bcast15/31 fold the four
// rows into lane 63, which is broadcast with readlane.
template <int ctrl, int row_mask> __device__ __forceinline__ float dpp_add(float v)
{
    return v + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), ctrl, row_mask, 0xF, false));
}
__device__ __forceinline__ float wave_sum_dpp(float v)
{
    v = dpp_add<0xB1, 0xF>(v);  // quad_perm [1,0,3,2]
    v = dpp_add<0x4E, 0xF>(v);  // quad_perm [2,3,0,1]
    v = dpp_add<0x141, 0xF>(v); // row_half_mirror
    v = dpp_add<0x140, 0xF>(v); // row_mirror
    v = dpp_add<0x142, 0xA>(v); // row_bcast:15 -> rows 1, 3
    v = dpp_add<0x143, 0xC>(v); // row_bcast:31 -> rows 2, 3
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}

// sum over aligned groups of `lpk` lanes (1, 2, 4, 8 or 16) with in-row DPP; every lane gets its group's sum
__device__ __forceinline__ float group_sum(float v, uint32_t lpk)
{
    if (lpk >= 2)
        v = dpp_add<0xB1, 0xF>(v); // quad_perm [1,0,3,2]
    if (lpk >= 4)
        v = dpp_add<0x4E, 0xF>(v); // quad_perm [2,3,0,1]
    if (lpk >= 8)
        v = dpp_add<0x141, 0xF>(v); // row_half_mirror
    if (lpk >= 16)
        v = dpp_add<0x140, 0xF>(v); // row_mirror
    return v;
}

template <int ctrl, int row_mask> __device__ __forceinline__ float dpp_max(float v)
{
    return fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(v), __float_as_int(v), ctrl, row_mask,
                                                               0xF, false)));
}
__device__ __forceinline__ float wave_max_dpp(float v)
{
    v = dpp_max<0xB1, 0xF>(v);
    v = dpp_max<0x4E, 0xF>(v);
    v = dpp_max<0x141, 0xF>(v);
    v = dpp_max<0x140, 0xF>(v);
    v = dpp_max<0x142, 0xA>(v);
    v = dpp_max<0x143, 0xC>(v);
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}

// reductions over the 4 waves of a 256-thread block; `red` holds 4 floats and is not reused by the other one
__device__ __forceinline__ float block4_max(float v, float *red)
{
    v = wave_max_dpp(v);
    if ((threadIdx.x & 63) == 0)
        red[threadIdx.x >> 6] = v;
    __syncthreads();
    return fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
}
__device__ __forceinline__ float block4_sum(float v, float *red)
{
    v = wave_sum_dpp(v);
    if ((threadIdx.x & 63) == 0)
        red[threadIdx.x >> 6] = v;
    __syncthreads();
    return (red[0] + red[1]) + (red[2] + red[3]);
}

// RoPE rotation terms c v0 - s v1 and s v0 + c v1 (src/shaders/vkllm_rope.comp:72-75) with every product and sum
// rounded on its own (no fused multiply-add)
__device__ __forceinline__ float rope_mul_sub(float c, float a, float s, float b)
{
    return __fsub_rn(__fmul_rn(c, a), __fmul_rn(s, b));
}
__device__ __forceinline__ float rope_mul_add(float s, float a, float c, float b)
{
    return __fadd_rn(__fmul_rn(s, a), __fmul_rn(c, b));
}

} // namespace vk
