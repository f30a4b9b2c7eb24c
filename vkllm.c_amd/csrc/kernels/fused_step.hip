// Fused gfx950 kernels of the LLaMA-2 token step (src/models/vkllm_llama2_layers.c:13-354 as fused stages).
//
// Every stage rounds to fp16 exactly where the reference's graph materialises an fp16 tensor (norm output,
// Q/K/V, RoPE output, scores, probabilities, attention output, projection outputs, residual sums, SiLU(gate),
// up*gate, logits), so fusing changes only fp32 summation order.
//
// Decode (one token) runs five kernels per layer:
//   gemv<QKV>      RMSNorm prologue, [Wq;Wk;Wv] rows, RoPE on q/k, k/v appended to the caches
//   attn_decode    scores, softmax and P.V for each head, one kernel, no cross-workgroup merge
//   gemv<RESID>    Wo rows, residual add in place
//   gemv<GATEUP>   RMSNorm prologue, up and gate rows side by side, SiLU(gate)*up
//   gemv<RESID>    Wd rows, residual add in place
#include <float.h>

#include "device_common.h"
#include "kernels.h"

namespace vk
{

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

// ---------------------------------------------------------------------------------------------------------------
// EMBEDDING (src/shaders/vkllm_embedding.comp:138-167) for contiguous rows
__global__ void embed_rows_kernel(const uint32_t *toks, const uint16_t *embd, uint16_t *h, uint32_t V, uint32_t D,
                                  uint32_t unk)
{
    const uint32_t s = blockIdx.x;
    uint32_t tok = toks[s];
    if (tok >= V)
        tok = unk;
    u32x4 *dst = (u32x4 *)(h + (size_t)s * D);
    const uint32_t nv = D / 8;
    if (tok >= V)
    {
        for (uint32_t i = threadIdx.x; i < nv; i += blockDim.x)
            dst[i] = (u32x4){0, 0, 0, 0};
        return;
    }
    const u32x4 *src = (const u32x4 *)(embd + (size_t)tok * D);
    for (uint32_t i = threadIdx.x; i < nv; i += blockDim.x)
        dst[i] = src[i];
}

hipError_t launch_embed_rows(hipStream_t st, const uint32_t *toks, uint32_t S, const uint16_t *embd, uint16_t *h,
                             uint32_t V, uint32_t D, uint32_t unk)
{
    embed_rows_kernel<<<S, 128, 0, st>>>(toks, embd, h, V, D, unk);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------------------------------------------
// RMSNORM (src/shaders/vkllm_rmsnorm.comp:31-82): y = fp16((x * w) * (1 / sqrt(sum(x^2) / D + eps)))

// normalises row `x` (D fp16) into `dst` (8 halfs per u32x4); all threads of the block take part
__device__ __forceinline__ void rmsnorm_row_to(const uint16_t *x, const float *w, u32x4 *dst, uint32_t D, float eps,
                                               float *red)
{
    const uint32_t nv = D / 8;
    const u32x4 *xv = (const u32x4 *)x;
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
    const float4 *wv = (const float4 *)w;
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
        dst[i] = o;
    }
}

__global__ __launch_bounds__(256) void rmsnorm_rows_kernel(const uint16_t *x, const float *w, uint16_t *y, uint32_t D,
                                                           float eps)
{
    __shared__ float red[8];
    const size_t s = blockIdx.x;
    rmsnorm_row_to(x + s * D, w, (u32x4 *)(y + s * D), D, eps, red);
}

hipError_t launch_rmsnorm_rows(hipStream_t st, const uint16_t *x, const float *w, uint16_t *y, uint32_t S,
                               uint32_t D, float eps)
{
    rmsnorm_rows_kernel<<<S, 256, 0, st>>>(x, w, y, D, eps);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------------------------------------------
// GEMV: one wave per work unit (two weight rows), each lane streaming 16-byte slices of both rows against the
// input vector held in LDS, fp32 accumulation with widening FMAs, DPP wave reduction. Workgroups of four waves
// walk the units grid-stride so the prologue (input vector, optional RMSNorm) is paid once per workgroup.
constexpr int kGemvUnroll = 8;

__device__ __forceinline__ float rope_mul_sub(float c, float a, float s, float b)
{
    return __fsub_rn(__fmul_rn(c, a), __fmul_rn(s, b));
}
__device__ __forceinline__ float rope_mul_add(float s, float a, float c, float b)
{
    return __fadd_rn(__fmul_rn(s, a), __fmul_rn(c, b));
}

template <int EPI> __global__ __launch_bounds__(256) void gemv_kernel(GemvArgs a)
{
    extern __shared__ u32x4 xs[];
    __shared__ float red[8];
    const uint32_t lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
    const uint32_t nvec = a.K / 8;

    if (a.norm_w)
        rmsnorm_row_to(a.x, a.norm_w, xs, a.K, a.eps, red);
    else
        for (uint32_t i = threadIdx.x; i < nvec; i += blockDim.x)
            xs[i] = ((const u32x4 *)a.x)[i];
    __syncthreads();

    const uint32_t stride = gridDim.x * 4;
    for (uint32_t u = blockIdx.x * 4 + wid; u < a.units; u += stride)
    {
        uint32_t r0, r1;
        if (EPI == EPI_GATEUP)
        {
            r0 = u;
            r1 = a.units + u;
        }
        else
        {
            r0 = 2 * u;
            r1 = 2 * u + 1;
        }
        const bool has1 = r1 < a.rows;
        const u32x4 *w0 = (const u32x4 *)(a.w + (size_t)r0 * a.K);
        const u32x4 *w1 = (const u32x4 *)(a.w + (size_t)(has1 ? r1 : r0) * a.K);
        float acc0 = 0.f, acc1 = 0.f;
        for (uint32_t v0 = lane; v0 < nvec; v0 += 64 * kGemvUnroll)
        {
            u32x4 wa[kGemvUnroll], wb[kGemvUnroll];
#pragma unroll
            for (int k = 0; k < kGemvUnroll; ++k)
            {
                const uint32_t vi = v0 + 64 * k;
                if (vi < nvec)
                {
                    wa[k] = __builtin_nontemporal_load(w0 + vi);
                    wb[k] = __builtin_nontemporal_load(w1 + vi);
                }
                else
                {
                    wa[k] = (u32x4){0, 0, 0, 0};
                    wb[k] = (u32x4){0, 0, 0, 0};
                }
            }
#pragma unroll
            for (int k = 0; k < kGemvUnroll; ++k)
            {
                const uint32_t vi = v0 + 64 * k;
                if (vi < nvec)
                {
                    const u32x4 xv = xs[vi];
                    acc0 = dot8(wa[k], xv, acc0);
                    acc1 = dot8(wb[k], xv, acc1);
                }
            }
        }
        acc0 = wave_sum_dpp(acc0);
        acc1 = wave_sum_dpp(acc1);
        if (lane != 0)
            continue;
        if (EPI == EPI_PLAIN)
        {
            a.out[r0] = f2h(acc0);
            if (has1)
                a.out[r1] = f2h(acc1);
        }
        else if (EPI == EPI_RESID)
        {
            a.out[r0] = f2h(h2f(a.resid[r0]) + h2f(f2h(acc0)));
            if (has1)
                a.out[r1] = f2h(h2f(a.resid[r1]) + h2f(f2h(acc1)));
        }
        else if (EPI == EPI_GATEUP)
        {
            const float up = h2f(f2h(acc0));
            const float gate = h2f(f2h(silu(acc1)));
            a.out[u] = f2h(up * gate);
        }
        else // EPI_QKV: rows r0 (even) and r1 = r0 + 1 of the same head
        {
            const uint32_t region = r0 / a.D, rr = r0 % a.D, head = rr / a.hd, dim = rr % a.hd;
            const float v0 = h2f(f2h(acc0)), v1 = h2f(f2h(acc1));
            const uint32_t pos = a.step->offset;
            const size_t cache = ((size_t)head * a.ctx + pos) * a.hd + dim;
            if (region == 2)
            {
                a.vc[cache] = f2h(v0);
                a.vc[cache + 1] = f2h(v1);
            }
            else
            {
                const float f = (float)pos / a.freqs[dim / 2];
                const float c = cosf(f), s = sinf(f);
                const uint16_t o0 = f2h(rope_mul_sub(c, v0, s, v1)), o1 = f2h(rope_mul_add(s, v0, c, v1));
                if (region == 0)
                {
                    a.out[rr] = o0;
                    a.out[rr + 1] = o1;
                }
                else
                {
                    a.kc[cache] = o0;
                    a.kc[cache + 1] = o1;
                }
            }
        }
    }
}

hipError_t launch_gemv(hipStream_t st, int epi, const GemvArgs &a, int cu_count)
{
    if (a.K % 8 != 0 || a.units == 0)
        return hipErrorInvalidValue;
    uint32_t blocks = (a.units + 3) / 4;
    const uint32_t cap = (uint32_t)(cu_count > 0 ? cu_count : 256) * 4;
    blocks = blocks > cap ? cap : blocks;
    const size_t lds = (size_t)a.K * 2;
    switch (epi)
    {
    case EPI_PLAIN:
        gemv_kernel<EPI_PLAIN><<<blocks, 256, lds, st>>>(a);
        break;
    case EPI_RESID:
        gemv_kernel<EPI_RESID><<<blocks, 256, lds, st>>>(a);
        break;
    case EPI_GATEUP:
        gemv_kernel<EPI_GATEUP><<<blocks, 256, lds, st>>>(a);
        break;
    case EPI_QKV:
        gemv_kernel<EPI_QKV><<<blocks, 256, lds, st>>>(a);
        break;
    default:
        return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

// ---------------------------------------------------------------------------------------------------------------
// Attention for one query row of one head (src/models/vkllm_llama2_layers.c:223-257 with
// src/shaders/vkllm_softmax.comp:42-96): s_j = fp16(scale * q.k_j), j < kv; p = fp16(exp(s - max) / sum);
// out[d] = fp16(sum_j p_j V[j][d]) for d in [d0, d0 + dn); with `transposed`, out[n] = fp16(sum_k p_k V[n][k]).
// `sm` holds kv floats. All 256 threads of the block take part.
__device__ void attn_row(const uint16_t *q, const uint16_t *K, const uint16_t *V, uint16_t *out, uint32_t kv,
                         uint32_t hd, float scale, bool transposed, uint32_t d0, uint32_t dn, float *sm, float *red,
                         float *part)
{
    const uint32_t tid = threadIdx.x;
    const uint32_t vpr = hd / 8; // 16-byte vectors per cache row
    uint32_t lpk = 1;            // lanes per key: power of two >= vpr
    while (lpk < vpr)
        lpk <<= 1;
    const uint32_t kl = tid % lpk, ks = tid / lpk, kpi = 256 / lpk;
    u32x4 qv = (u32x4){0, 0, 0, 0};
    if (kl < vpr)
        qv = ((const u32x4 *)q)[kl];
    constexpr int U = 4;
    for (uint32_t j0 = ks; j0 < kv; j0 += kpi * U)
    {
        u32x4 kvec[U];
#pragma unroll
        for (int t = 0; t < U; ++t)
        {
            const uint32_t j = j0 + kpi * t;
            kvec[t] = (kl < vpr && j < kv) ? ((const u32x4 *)(K + (size_t)j * hd))[kl] : (u32x4){0, 0, 0, 0};
        }
#pragma unroll
        for (int t = 0; t < U; ++t)
        {
            float p = dot8(kvec[t], qv, 0.f);
            for (uint32_t o = lpk / 2; o > 0; o >>= 1)
                p += __shfl_xor(p, (int)o, (int)lpk);
            const uint32_t j = j0 + kpi * t;
            if (kl == 0 && j < kv)
                sm[j] = h2f(f2h(p * scale));
        }
    }
    __syncthreads();
    float mx = -FLT_MAX;
    for (uint32_t j = tid; j < kv; j += 256)
        mx = fmaxf(mx, sm[j]);
    mx = block_max(mx, red);
    float sum = 0.f;
    for (uint32_t j = tid; j < kv; j += 256)
        sum += expf(sm[j] - mx);
    sum = block_sum(sum, red);
    for (uint32_t j = tid; j < kv; j += 256)
        sm[j] = h2f(f2h(expf(sm[j] - mx) / sum));
    __syncthreads();

    if (transposed)
    {
        for (uint32_t n = d0 + tid; n < d0 + dn; n += 256)
        {
            const uint16_t *row = V + (size_t)n * hd;
            float acc = 0.f;
            for (uint32_t k = 0; k < kv; ++k)
                acc = fmaf(sm[k], h2f(row[k]), acc);
            out[n] = f2h(acc);
        }
        return;
    }
    const uint32_t vps = dn / 8;        // vectors of this block's slice per row
    const uint32_t rpi = 256 / vps;     // rows per iteration
    const uint32_t r = tid / vps, c = tid % vps;
    float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    if (r < rpi)
    {
        for (uint32_t j0 = r; j0 < kv; j0 += rpi * U)
        {
            u32x4 vv[U];
#pragma unroll
            for (int t = 0; t < U; ++t)
            {
                const uint32_t j = j0 + rpi * t;
                vv[t] = j < kv ? ((const u32x4 *)(V + (size_t)j * hd + d0))[c] : (u32x4){0, 0, 0, 0};
            }
#pragma unroll
            for (int t = 0; t < U; ++t)
            {
                const uint32_t j = j0 + rpi * t;
                const float p = j < kv ? sm[j] : 0.f;
#pragma unroll
                for (int e = 0; e < 4; ++e)
                {
                    acc[2 * e] = fmaf(p, half_lo(vv[t][e]), acc[2 * e]);
                    acc[2 * e + 1] = fmaf(p, half_hi(vv[t][e]), acc[2 * e + 1]);
                }
            }
        }
#pragma unroll
        for (int e = 0; e < 8; ++e)
            part[r * dn + c * 8 + e] = acc[e];
    }
    __syncthreads();
    for (uint32_t d = tid; d < dn; d += 256)
    {
        float s = 0.f;
        for (uint32_t k = 0; k < rpi; ++k)
            s += part[k * dn + d];
        out[d0 + d] = f2h(s);
    }
}

// grid: H * groups workgroups; the `groups` workgroups of a head each produce hd/groups output dims (and all
// recompute the head's scores); block ids are arranged so they share blockIdx % 8, i.e. one XCD and its L2.
__global__ __launch_bounds__(256) void attn_decode_kernel(const uint16_t *q, const uint16_t *kc, const uint16_t *vc,
                                                          uint16_t *out, const Step *step, uint32_t H, uint32_t hd,
                                                          uint32_t ctx, float scale, uint32_t groups)
{
    extern __shared__ float sm[];
    __shared__ float red[8];
    __shared__ float part[2048];
    const uint32_t b = blockIdx.x;
    const uint32_t head = (b % 8) + 8 * (b / (8 * groups)), g = (b / 8) % groups;
    if (head >= H)
        return;
    const uint32_t kv = step->offset + 1;
    const uint32_t dn = hd / groups;
    const size_t hoff = (size_t)head * ctx * hd;
    attn_row(q + (size_t)head * hd, kc + hoff, vc + hoff, out + (size_t)head * hd, kv, hd, scale, kv == hd, g * dn, dn,
             sm, red, part);
}

hipError_t launch_attn_decode(hipStream_t st, const uint16_t *q, const uint16_t *kc, const uint16_t *vc,
                              uint16_t *out, const Step *step, uint32_t H, uint32_t hd, uint32_t ctx, float scale)
{
    if (hd % 8 != 0 || hd > 256)
        return hipErrorInvalidValue;
    // dims per group stay a multiple of 8 and the reduction buffer fits: rows-per-iteration * dims <= 2048
    uint32_t groups = 1;
    const uint32_t vpr = hd / 8;
    for (uint32_t g = 8; g > 1; --g)
        if (vpr % g == 0 && H * g <= 256)
        {
            groups = g;
            break;
        }
    const uint32_t heads8 = (H + 7) / 8 * 8;
    const uint32_t blocks = heads8 * groups;
    const size_t lds = (size_t)ctx * sizeof(float);
    attn_decode_kernel<<<blocks, 256, lds, st>>>(q, kc, vc, out, step, H, hd, ctx, scale, groups);
    return hipGetLastError();
}

// prefill: one workgroup per (query row, head); the transposition rule applies when the step's kv == hd
__global__ __launch_bounds__(256) void attn_prefill_kernel(const uint16_t *q, const uint16_t *kc, const uint16_t *vc,
                                                           uint16_t *out, uint32_t offset, uint32_t S, uint32_t H,
                                                           uint32_t hd, uint32_t ctx, float scale)
{
    extern __shared__ float sm[];
    __shared__ float red[8];
    __shared__ float part[2048];
    const uint32_t s = blockIdx.x, head = blockIdx.y;
    const uint32_t D = H * hd;
    const size_t hoff = (size_t)head * ctx * hd;
    const bool transposed = offset + S == hd;
    attn_row(q + (size_t)s * D + (size_t)head * hd, kc + hoff, vc + hoff, out + (size_t)s * D + (size_t)head * hd,
             offset + s + 1, hd, scale, transposed, 0, hd, sm, red, part);
}

hipError_t launch_attn_prefill(hipStream_t st, const uint16_t *q, const uint16_t *kc, const uint16_t *vc,
                               uint16_t *out, uint32_t offset, uint32_t S, uint32_t H, uint32_t hd, uint32_t ctx,
                               float scale)
{
    if (hd % 8 != 0 || hd > 256)
        return hipErrorInvalidValue;
    const size_t lds = (size_t)(offset + S) * sizeof(float);
    attn_prefill_kernel<<<dim3(S, H), 256, lds, st>>>(q, kc, vc, out, offset, S, H, hd, ctx, scale);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------------------------------------------
// RoPE (normal style, src/shaders/vkllm_rope.comp:146-174) on q and k of a prefill QKV block, k and v appended to
// the caches (src/shaders/vkllm_update_rows.comp:21-46)
__global__ void rope_kv_kernel(const uint16_t *qkv, uint16_t *q, uint16_t *kc, uint16_t *vc, const float *freqs,
                               uint32_t offset, uint32_t S, uint32_t D, uint32_t hd, uint32_t ctx)
{
    const uint32_t pairs = D / 2;
    const uint64_t total = (uint64_t)S * pairs;
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += (uint64_t)gridDim.x * blockDim.x)
    {
        const uint32_t s = (uint32_t)(i / pairs), p = (uint32_t)(i % pairs);
        const uint32_t col = 2 * p, head = col / hd, dim = col % hd;
        const uint32_t pos = offset + s;
        const uint16_t *row = qkv + (size_t)s * 3 * D;
        const float f = (float)pos / freqs[dim / 2];
        const float c = cosf(f), sn = sinf(f);
        const float q0 = h2f(row[col]), q1 = h2f(row[col + 1]);
        const float k0 = h2f(row[D + col]), k1 = h2f(row[D + col + 1]);
        q[(size_t)s * D + col] = f2h(rope_mul_sub(c, q0, sn, q1));
        q[(size_t)s * D + col + 1] = f2h(rope_mul_add(sn, q0, c, q1));
        const size_t cache = ((size_t)head * ctx + pos) * hd + dim;
        kc[cache] = f2h(rope_mul_sub(c, k0, sn, k1));
        kc[cache + 1] = f2h(rope_mul_add(sn, k0, c, k1));
        vc[cache] = row[2 * D + col];
        vc[cache + 1] = row[2 * D + col + 1];
    }
}

hipError_t launch_rope_kv(hipStream_t st, const uint16_t *qkv, uint16_t *q, uint16_t *kc, uint16_t *vc,
                          const float *freqs, uint32_t offset, uint32_t S, uint32_t D, uint32_t hd, uint32_t ctx)
{
    const uint64_t total = (uint64_t)S * (D / 2);
    uint32_t grid = (uint32_t)((total + 255) / 256);
    grid = grid > 16384 ? 16384 : grid;
    rope_kv_kernel<<<grid, 256, 0, st>>>(qkv, q, kc, vc, freqs, offset, S, D, hd, ctx);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------------------------------------------
// up * SiLU(gate) (src/models/vkllm_llama2_layers.c:54-60, BIN op 2) on a [S, 2F] block whose gate half already
// holds fp16(silu(gate))
__global__ void swiglu_kernel(const uint16_t *ug, uint16_t *act, uint32_t S, uint32_t F)
{
    const uint64_t total = (uint64_t)S * F;
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += (uint64_t)gridDim.x * blockDim.x)
    {
        const uint64_t s = i / F, n = i % F;
        const uint16_t *row = ug + s * 2 * F;
        act[i] = f2h(h2f(row[n]) * h2f(row[F + n]));
    }
}

hipError_t launch_swiglu(hipStream_t st, const uint16_t *ug, uint16_t *act, uint32_t S, uint32_t F)
{
    const uint64_t total = (uint64_t)S * F;
    uint32_t grid = (uint32_t)((total + 255) / 256);
    grid = grid > 16384 ? 16384 : grid;
    swiglu_kernel<<<grid, 256, 0, st>>>(ug, act, S, F);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------------------------------------------
// ARG_MAX with the reference's tie rule (src/shaders/vkllm_arg_max.comp:40-97), 1024 threads per row: thread t
// sees elements i == t (mod 1024), all in lane t % 32 of the reference's 32-lane scan; lane partials merge by
// (larger value, then smaller index); the 32 lanes then fold with the strict-'>' tree (lower lane keeps ties).
__global__ __launch_bounds__(1024) void argmax_rows_kernel(const uint16_t *logits, uint32_t *ids, uint32_t V)
{
    __shared__ float sv[1024];
    __shared__ uint32_t si[1024];
    __shared__ int sh[1024];
    const uint32_t t = threadIdx.x;
    const uint16_t *row = logits + (size_t)blockIdx.x * V;
    float bv = -FLT_MAX;
    uint32_t bi = t % 32;
    int have = 0;
    if (t < 32)
    {
        have = 1;
        if (t < V)
            bv = h2f(row[t]);
    }
    for (uint32_t i = (t < 32 ? t + 1024 : t); i < V; i += 1024)
    {
        const float v = h2f(row[i]);
        if (!have || v > bv)
        {
            bv = v;
            bi = i;
            have = 1;
        }
    }
    sv[t] = bv;
    si[t] = bi;
    sh[t] = have;
    __syncthreads();
    if (t < 32)
    {
        for (uint32_t k = t + 32; k < 1024; k += 32)
        {
            if (!sh[k])
                continue;
            if (sv[k] > bv || (sv[k] == bv && si[k] < bi))
            {
                bv = sv[k];
                bi = si[k];
            }
        }
        sv[t] = bv;
        si[t] = bi;
    }
    __syncthreads();
    if (t == 0)
    {
        for (uint32_t s = 16; s > 0; s >>= 1)
            for (uint32_t l = 0; l < s; ++l)
                if (sv[l + s] > sv[l])
                {
                    sv[l] = sv[l + s];
                    si[l] = si[l + s];
                }
        ids[blockIdx.x] = si[0];
    }
}

hipError_t launch_argmax_rows(hipStream_t st, const uint16_t *logits, uint32_t *ids, uint32_t S, uint32_t V)
{
    argmax_rows_kernel<<<S, 1024, 0, st>>>(logits, ids, V);
    return hipGetLastError();
}

} // namespace vk
