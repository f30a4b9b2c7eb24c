// Fused gfx950 kernels of the LLaMA-2 token step (src/models/vkllm_llama2_layers.c:13-354 as fused stages).
//
// Every stage rounds to fp16 exactly where the reference's graph materialises an fp16 tensor (norm output,
// Q/K/V, RoPE output, scores, probabilities, attention output, projection outputs, residual sums, SiLU(gate),
// up*gate, logits), so fusing changes only fp32 summation order.
//
// Decode (one token) runs six kernels per layer:
//   gemv<QKV>      RMSNorm prologue, [Wq;Wk;Wv] rows, RoPE on q/k, k/v appended to the caches
//   attn_scores    scores and per-chunk softmax statistics, split over the cache positions
//   attn_pv        probabilities with the row's statistics, P.V per chunk, chunk merge by the last block
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

// first kernel of a single-token step: position and token from the pinned host block
__global__ void embed_decode_kernel(const DecodeIo *io, Step *step, const uint16_t *embd, uint16_t *h, uint32_t V,
                                    uint32_t D, uint32_t unk)
{
    const uint32_t offset = io->offset;
    uint32_t tok = io->token;
    if (threadIdx.x == 0)
    {
        step->offset = offset;
        step->S = 1;
    }
    if (tok >= V)
        tok = unk;
    u32x4 *dst = (u32x4 *)h;
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

hipError_t launch_embed_decode(hipStream_t st, const DecodeIo *io, Step *step, const uint16_t *embd, uint16_t *h,
                               uint32_t V, uint32_t D, uint32_t unk)
{
    if (D % 8 != 0)
        return hipErrorInvalidValue;
    embed_decode_kernel<<<1, 256, 0, st>>>(io, step, embd, h, V, D, unk);
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
                // unconditional loads at clamped addresses; the slots past the row are skipped below
                const uint32_t vi = min(v0 + 64 * k, nvec - 1);
                wa[k] = __builtin_nontemporal_load(w0 + vi);
                wb[k] = __builtin_nontemporal_load(w1 + vi);
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

hipError_t launch_gemv_loop(hipStream_t st, int epi, const GemvArgs &a, int cu_count)
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

// GEMV with the input prologue overlapped by the weight stream. A wave owns units of R weight rows (R/2 up rows
// next to R/2 gate rows for EPI_GATEUP; R even for EPI_QKV so RoPE pairs stay together); lane l holds the 16-byte
// vectors l + 64 i (i < NV) of each row, so NV * 512 >= K. Order of work in a workgroup:
//   1. its threads' share of the input vector (and of the RMSNorm weights) into registers
//   2. the weight vectors of each wave's first unit: the bulk of the traffic is in flight from here on
//   3. RMSNorm over the registers (block reduction in LDS), the normalised input into LDS
//   4. per unit: dot products against LDS, the next unit's weights issued before this unit's reduction
// Vector-memory counters retire in issue order, so waiting for the input (issued first) never waits for weights.
template <int EPI> __device__ __forceinline__ void gemv_rows_of(const GemvArgs &a, uint32_t u, int R, uint32_t *rows)
{
    for (int k = 0; k < R; ++k)
    {
        if (EPI == EPI_GATEUP)
            rows[k] = k < R / 2 ? (R / 2) * u + k : a.rows / 2 + (R / 2) * u + (k - R / 2);
        else
            rows[k] = R * u + k;
    }
}

template <int EPI, int R> __device__ __forceinline__ void gemv_epilogue(const GemvArgs &a, uint32_t u,
                                                                        const uint32_t *rows, const float *acc)
{
    if (EPI == EPI_PLAIN)
    {
#pragma unroll
        for (int k = 0; k < R; ++k)
            if (rows[k] < a.rows)
                a.out[rows[k]] = f2h(acc[k]);
    }
    else if (EPI == EPI_RESID)
    {
#pragma unroll
        for (int k = 0; k < R; ++k)
            if (rows[k] < a.rows)
                a.out[rows[k]] = f2h(h2f(a.resid[rows[k]]) + h2f(f2h(acc[k])));
    }
    else if (EPI == EPI_GATEUP)
    {
#pragma unroll
        for (int k = 0; k < R / 2; ++k)
        {
            const float up = h2f(f2h(acc[k]));
            const float gate = h2f(f2h(silu(acc[k + R / 2])));
            a.out[(R / 2) * u + k] = f2h(up * gate);
        }
    }
    else // EPI_QKV: rows (r, r + 1), r even, are one RoPE pair of one head
    {
        const uint32_t pos = a.step->offset;
#pragma unroll
        for (int k = 0; k < R; k += 2)
        {
            const uint32_t r0 = rows[k];
            if (r0 >= a.rows)
                continue;
            const uint32_t region = r0 / a.D, rr = r0 % a.D, head = rr / a.hd, dim = rr % a.hd;
            const float v0 = h2f(f2h(acc[k])), v1 = h2f(f2h(acc[k + 1]));
            const size_t cache = ((size_t)head * a.ctx + pos) * a.hd + dim;
            if (region == 2)
            {
                a.vc[cache] = f2h(v0);
                a.vc[cache + 1] = f2h(v1);
                continue;
            }
            const float f = (float)pos / a.freqs[dim / 2];
            const float c = cosf(f), sn = sinf(f);
            const uint16_t o0 = f2h(rope_mul_sub(c, v0, sn, v1)), o1 = f2h(rope_mul_add(sn, v0, c, v1));
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

template <int EPI, int R, int NV> __global__ __launch_bounds__(256) void gemv_fast_kernel(GemvArgs a, uint32_t units)
{
    extern __shared__ u32x4 xs[];
    __shared__ float red[8];
    constexpr int XV = (NV * 64 + 255) / 256; // input vectors per thread
    const uint32_t tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
    const uint32_t nvec = a.K / 8;
    const bool norm = a.norm_w != nullptr;

    // 1. input share (and RMSNorm weights)
    // Loads are unconditional at clamped addresses (a guarded load compiles to a branch and a full wait per load);
    // lanes past the end read a valid duplicate that is masked out below.
    u32x4 xr[XV];
    float4 nw[XV][2];
    const float4 *nwp = (const float4 *)(norm ? a.norm_w : (const float *)a.x);
#pragma unroll
    for (int i = 0; i < XV; ++i)
    {
        const uint32_t vi = min(tid + 256 * i, nvec - 1);
        xr[i] = ((const u32x4 *)a.x)[vi];
        if (norm)
        {
            nw[i][0] = nwp[2 * vi];
            nw[i][1] = nwp[2 * vi + 1];
        }
    }
#pragma unroll
    for (int i = 0; i < XV; ++i)
        if (tid + 256 * i >= nvec)
            xr[i] = (u32x4){0, 0, 0, 0};

    // 2. first unit's weights
    const uint32_t stride = gridDim.x * 4;
    uint32_t u = blockIdx.x * 4 + wid;
    u32x4 w[R][NV];
    uint32_t rows[R];
    auto load_unit = [&](uint32_t unit) {
        gemv_rows_of<EPI>(a, unit, R, rows);
#pragma unroll
        for (int k = 0; k < R; ++k)
        {
            // rows past the end (or of units past the end) read row 0; their sums are never stored
            const bool ok = unit < units && rows[k] < a.rows;
            const u32x4 *wr = (const u32x4 *)(a.w + (size_t)(ok ? rows[k] : 0) * a.K);
#pragma unroll
            for (int i = 0; i < NV; ++i)
                w[k][i] = __builtin_nontemporal_load(wr + min(lane + 64 * i, nvec - 1));
        }
    };
    load_unit(u);

    // 3. prologue
    if (norm)
    {
        float ss = 0.f;
#pragma unroll
        for (int i = 0; i < XV; ++i)
#pragma unroll
            for (int k = 0; k < 4; ++k)
            {
                const float lo = half_lo(xr[i][k]), hi = half_hi(xr[i][k]);
                ss += lo * lo;
                ss += hi * hi;
            }
        ss = block_sum(ss, red);
        const float alpha = 1.0f / sqrtf(ss / (float)a.K + a.eps);
#pragma unroll
        for (int i = 0; i < XV; ++i)
        {
            const float ws[8] = {nw[i][0].x, nw[i][0].y, nw[i][0].z, nw[i][0].w,
                                 nw[i][1].x, nw[i][1].y, nw[i][1].z, nw[i][1].w};
#pragma unroll
            for (int k = 0; k < 4; ++k)
            {
                const float lo = half_lo(xr[i][k]), hi = half_hi(xr[i][k]);
                xr[i][k] = pack2(f2h((lo * ws[2 * k]) * alpha), f2h((hi * ws[2 * k + 1]) * alpha));
            }
        }
    }
#pragma unroll
    for (int i = 0; i < XV; ++i)
    {
        const uint32_t vi = tid + 256 * i;
        if (vi < nvec)
            xs[vi] = xr[i];
    }
    __syncthreads();

    // 4. units
    while (u < units)
    {
        float acc[R];
#pragma unroll
        for (int k = 0; k < R; ++k)
            acc[k] = 0.f;
#pragma unroll
        for (int i = 0; i < NV; ++i)
        {
            const uint32_t vi = lane + 64 * i;
            if (vi < nvec)
            {
                const u32x4 xv = xs[vi];
#pragma unroll
                for (int k = 0; k < R; ++k)
                    acc[k] = dot8(w[k][i], xv, acc[k]);
            }
        }
        uint32_t cur_rows[R];
#pragma unroll
        for (int k = 0; k < R; ++k)
            cur_rows[k] = rows[k];
        const uint32_t cur = u;
        u += stride;
        if (u < units)
            load_unit(u);
#pragma unroll
        for (int k = 0; k < R; ++k)
            acc[k] = wave_sum_dpp(acc[k]);
        if (lane == 0)
            gemv_epilogue<EPI, R>(a, cur, cur_rows, acc);
    }
}

// units of R rows for `a`; 0 when R does not fit the epilogue's pairing
static uint32_t gemv_units(int epi, const GemvArgs &a, int R)
{
    if (epi == EPI_GATEUP)
        return (R % 2 == 0 && a.rows % R == 0) ? a.rows / R : 0;
    if (epi == EPI_QKV && R % 2 != 0)
        return 0;
    return (a.rows + R - 1) / R;
}

template <int EPI, int R, int NV> static hipError_t launch_fast(hipStream_t st, const GemvArgs &a, int cu_count)
{
    const uint32_t units = gemv_units(EPI, a, R);
    if (units == 0)
        return hipErrorInvalidValue;
    // resident workgroups per CU at this kernel's register use and this K's LDS, cached for the last K seen
    static size_t cached_lds = 0;
    static int per_cu = 0;
    const size_t lds = (size_t)a.K * 2;
    if (lds != cached_lds)
    {
        int n = 0;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, gemv_fast_kernel<EPI, R, NV>, 256, lds) != hipSuccess)
            n = 1;
        per_cu = n > 0 ? n : 1;
        cached_lds = lds;
    }
    uint32_t blocks = (units + 3) / 4;
    const uint32_t cap = (uint32_t)(cu_count > 0 ? cu_count : 256) * (uint32_t)per_cu;
    blocks = blocks > cap ? cap : blocks;
    gemv_fast_kernel<EPI, R, NV><<<blocks, 256, lds, st>>>(a, units);
    return hipGetLastError();
}

// smallest compiled NV >= the vectors each lane needs per row (nvec / 64), per R; 0 when none fits
static int gemv_pick_nv(int R, uint32_t nvec)
{
    static const int nv1[] = {2, 4, 8, 12, 16, 22, 28}, nv2[] = {2, 4, 8, 12, 14, 22}, nv4[] = {2, 4, 8};
    const int *t = R == 1 ? nv1 : R == 2 ? nv2 : nv4;
    const int n = R == 1 ? 7 : R == 2 ? 6 : 3;
    for (int i = 0; i < n; ++i)
        if ((uint32_t)t[i] * 64 >= nvec)
            return t[i];
    return 0;
}

#define GEMV_NV_CASE(R_, NV_)                                                                                       \
    case NV_:                                                                                                       \
        return launch_fast<EPI, R_, NV_>(st, a, cu_count)

template <int EPI> static hipError_t launch_epi(hipStream_t st, const GemvArgs &a, int cu_count, int R, int NV)
{
    if (R == 1)
        switch (NV)
        {
            GEMV_NV_CASE(1, 2);
            GEMV_NV_CASE(1, 4);
            GEMV_NV_CASE(1, 8);
            GEMV_NV_CASE(1, 12);
            GEMV_NV_CASE(1, 16);
            GEMV_NV_CASE(1, 22);
            GEMV_NV_CASE(1, 28);
        }
    if (R == 2)
        switch (NV)
        {
            GEMV_NV_CASE(2, 2);
            GEMV_NV_CASE(2, 4);
            GEMV_NV_CASE(2, 8);
            GEMV_NV_CASE(2, 12);
            GEMV_NV_CASE(2, 14);
            GEMV_NV_CASE(2, 22);
        }
    if (R == 4)
        switch (NV)
        {
            GEMV_NV_CASE(4, 2);
            GEMV_NV_CASE(4, 4);
            GEMV_NV_CASE(4, 8);
        }
    return hipErrorInvalidValue;
}
#undef GEMV_NV_CASE

// rows per unit: the number of 16-byte vectors each lane keeps in flight is R * NV
static int gemv_default_r(int epi, uint32_t K)
{
    (void)K;
    return epi == EPI_GATEUP || epi == EPI_QKV ? 2 : 1;
}

hipError_t launch_gemv(hipStream_t st, int epi, const GemvArgs &a, int cu_count)
{
    if (a.K % 8 != 0 || a.rows == 0)
        return hipErrorInvalidValue;
    const uint32_t nvec = a.K / 8;
    int R = a.rows_per_unit ? (int)a.rows_per_unit : gemv_default_r(epi, a.K);
    if (R == 1 && (epi == EPI_GATEUP || epi == EPI_QKV))
        R = 2;
    const int NV = (R == 1 || R == 2 || R == 4) ? gemv_pick_nv(R, nvec) : 0;
    if (NV != 0 && (epi != EPI_GATEUP || a.rows % R == 0))
    {
        switch (epi)
        {
        case EPI_PLAIN:
            return launch_epi<EPI_PLAIN>(st, a, cu_count, R, NV);
        case EPI_RESID:
            return launch_epi<EPI_RESID>(st, a, cu_count, R, NV);
        case EPI_GATEUP:
            return launch_epi<EPI_GATEUP>(st, a, cu_count, R, NV);
        case EPI_QKV:
            return launch_epi<EPI_QKV>(st, a, cu_count, R, NV);
        default:
            return hipErrorInvalidValue;
        }
    }
    return launch_gemv_loop(st, epi, a, cu_count);
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

// ---------------------------------------------------------------------------------------------------------------
// Decode attention. The reference materialises fp16 scores, fp16 probabilities and an fp16 attention output
// (src/models/vkllm_llama2_layers.c:223-257, src/shaders/vkllm_softmax.comp:42-96), so the probabilities are rounded
// with the GLOBAL max and sum of the row. Two kernels keep those rounding points without any cross-block merge:
//   attn_scores_kernel  split over the cache positions: chunk c of head h writes s_j = fp16(scale q.k_j) to the
//                       scores scratch and its chunk max m_c and l_c = sum_j exp(s_j - m_c)
//   attn_pv_kernel      split over the output dims: block (h, g) reduces M = max m_c, L = sum_c l_c exp(m_c - M)
//                       (the same reduction in every block of the head), then p_j = fp16(exp(s_j - M) / L) and
//                       out[d] = fp16(sum_j p_j v_j[d]) for its hd / G dims over all positions
// The chunk length (a multiple of 16 positions) follows kv on the device, so one captured graph serves every
// position. kv == hd takes the reference's transposed product p . V^T.

__device__ __forceinline__ void attn_chunks(uint32_t kv, uint32_t hd, uint32_t cmax, uint32_t &ch, uint32_t &nc)
{
    if (kv == hd)
    {
        ch = kv;
        nc = 1;
        return;
    }
    ch = (kv + cmax - 1) / cmax;
    ch = (ch + 15) / 16 * 16;
    nc = (kv + ch - 1) / ch;
}

// Lanes sharing one cache row when scoring keys: each lane takes two 16-byte vectors (16 dims) of the row.
__device__ __forceinline__ uint32_t key_lanes(uint32_t hd)
{
    uint32_t l = 1;
    while (l * 16 < hd)
        l <<= 1;
    return l;
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

// sm[j] = fp16(scale * q . K[j]) for j < n (K: n contiguous rows of hd halfs); all 256 threads take part. A key is
// scored by key_lanes(hd) lanes holding 16 dims each, U passes of keys in flight per thread, loads unconditional
// at clamped addresses. The lanes of one key share their loop trip count, so the group DPP sees only live lanes.
template <int U>
__device__ __forceinline__ void attn_score_keys(const uint16_t *q, const uint16_t *K, uint32_t n, uint32_t hd,
                                                float scale, float *sm)
{
    const uint32_t vpr = hd / 8, lpk = key_lanes(hd);
    const uint32_t tid = threadIdx.x, kl = tid % lpk, ks = tid / lpk, kpp = 256 / lpk;
    const uint32_t c0 = min(2 * kl, vpr - 1), c1 = min(2 * kl + 1, vpr - 1);
    const u32x4 *qv = (const u32x4 *)q;
    u32x4 q0 = qv[c0], q1 = qv[c1];
    if (2 * kl >= vpr)
        q0 = (u32x4){0, 0, 0, 0};
    if (2 * kl + 1 >= vpr)
        q1 = (u32x4){0, 0, 0, 0};
    const u32x4 *Kv = (const u32x4 *)K;
    for (uint32_t jb = ks; jb < n; jb += kpp * U)
    {
        u32x4 ka[U], kb[U];
#pragma unroll
        for (int t = 0; t < U; ++t)
        {
            const size_t row = (size_t)min(jb + kpp * t, n - 1) * vpr;
            ka[t] = Kv[row + c0];
            kb[t] = Kv[row + c1];
        }
#pragma unroll
        for (int t = 0; t < U; ++t)
        {
            float p = dot8(kb[t], q1, dot8(ka[t], q0, 0.f));
            p = group_sum(p, lpk);
            const uint32_t j = jb + kpp * t;
            if (kl == 0 && j < n)
                sm[j] = h2f(f2h(p * scale));
        }
    }
}

__global__ __launch_bounds__(256) void attn_scores_kernel(AttnDecodeArgs a)
{
    extern __shared__ float sm[]; // this chunk's scores
    __shared__ float rmax[4], rsum[4];
    const uint32_t h = blockIdx.x / a.cmax, c = blockIdx.x % a.cmax;
    const uint32_t kv = a.step->offset + 1;
    uint32_t ch, nc;
    attn_chunks(kv, a.hd, a.cmax, ch, nc);
    if (c >= nc)
        return;
    const uint32_t tid = threadIdx.x;
    const uint32_t j0 = c * ch, n = min(ch, kv - j0);
    // chunks hold a few dozen positions: two passes of keys per thread cover them
    attn_score_keys<2>(a.q + (size_t)h * a.hd, a.kc + ((size_t)h * a.ctx + j0) * a.hd, n, a.hd, a.scale, sm);
    __syncthreads();
    float mx = -FLT_MAX;
    for (uint32_t j = tid; j < n; j += 256)
        mx = fmaxf(mx, sm[j]);
    mx = block4_max(mx, rmax);
    float sum = 0.f;
    for (uint32_t j = tid; j < n; j += 256)
    {
        sum += expf(sm[j] - mx);
        a.scores[(size_t)h * a.ctx + j0 + j] = sm[j];
    }
    sum = block4_sum(sum, rsum);
    if (tid == 0)
    {
        a.stats[((size_t)h * a.cmax + c) * 2] = mx;
        a.stats[((size_t)h * a.cmax + c) * 2 + 1] = sum;
    }
}

// out[r] = fp16(sum_k p_k V[r][k]) for the block's rows r of the reference's transposed product (kv == hd)
__device__ __forceinline__ void attn_pv_transposed(const float *pl, const uint16_t *Vh, uint16_t *out, uint32_t kv,
                                                   uint32_t hd, uint32_t d0, uint32_t dg)
{
    for (uint32_t r = threadIdx.x; r < dg; r += 256)
    {
        const uint16_t *row = Vh + (size_t)(d0 + r) * hd;
        float acc = 0.f;
        for (uint32_t k = 0; k < kv; ++k)
            acc = fmaf(pl[k], h2f(row[k]), acc);
        out[r] = f2h(acc);
    }
}

// block b -> (head, dim group): the G blocks of a head get consecutive ids with equal b % 8, i.e. one XCD and its
// L2, so the partial lines of V rows that neighbouring groups read are fetched from HBM once
__device__ __forceinline__ void attn_block_head(uint32_t b, uint32_t G, uint32_t &h, uint32_t &g)
{
    h = (b % 8) + 8 * (b / (8 * G));
    g = (b / 8) % G;
}

__global__ __launch_bounds__(256) void attn_pv_kernel(AttnDecodeArgs a)
{
    __shared__ float rmax[4], rsum[4];
    __shared__ float part[2048];
    uint32_t h, g;
    attn_block_head(blockIdx.x, a.groups, h, g);
    if (h >= a.H)
        return;
    const uint32_t tid = threadIdx.x;
    const uint32_t kv = a.step->offset + 1;
    uint32_t ch, nc;
    attn_chunks(kv, a.hd, a.cmax, ch, nc);
    const float *st = a.stats + (size_t)h * a.cmax * 2;
    const float *S = a.scores + (size_t)h * a.ctx;
    const uint16_t *Vh = a.vc + (size_t)h * a.ctx * a.hd;
    const uint32_t dg = a.hd / a.groups, d0 = g * dg;
    uint16_t *out = a.out + (size_t)h * a.hd + d0;
    // loads in this order: chunk statistics, then V rows and scores, so waiting for the statistics (counters
    // retire in issue order) does not wait for V
    const uint32_t ci = min(tid, nc - 1);
    const float mc_raw = st[2 * ci], lc_raw = st[2 * ci + 1];
    const uint32_t lpr = dg / 8, vpr = a.hd / 8, rpp = 256 / lpr;
    const uint32_t kl = tid % lpr, ks = tid / lpr;
    const u32x4 *Vv = (const u32x4 *)Vh + d0 / 8 + kl;
    constexpr int U = 8;
    u32x4 vv[U];
    float sc[U];
#pragma unroll
    for (int t = 0; t < U; ++t)
    {
        const uint32_t j = min(ks + rpp * t, kv - 1);
        vv[t] = Vv[(size_t)j * vpr];
        sc[t] = S[j];
    }
    // softmax statistics of the whole row, reduced identically by every block of the head
    const float mc = tid < nc ? mc_raw : -FLT_MAX;
    const float M = block4_max(mc, rmax);
    const float L = block4_sum(tid < nc ? lc_raw * expf(mc - M) : 0.f, rsum);
    if (kv == a.hd)
    {
        float *pl = part;
        for (uint32_t j = tid; j < kv; j += 256)
            pl[j] = h2f(f2h(expf(S[j] - M) / L));
        __syncthreads();
        attn_pv_transposed(pl, Vh, out, kv, a.hd, d0, dg);
        return;
    }
    float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    for (uint32_t jb = ks; jb < kv; jb += rpp * U)
    {
        if (jb != ks)
        {
#pragma unroll
            for (int t = 0; t < U; ++t)
            {
                const uint32_t j = min(jb + rpp * t, kv - 1);
                vv[t] = Vv[(size_t)j * vpr];
                sc[t] = S[j];
            }
        }
#pragma unroll
        for (int t = 0; t < U; ++t)
        {
            const float pj = jb + rpp * t < kv ? h2f(f2h(expf(sc[t] - M) / L)) : 0.f;
#pragma unroll
            for (int e = 0; e < 4; ++e)
            {
                acc[2 * e] = fmaf(pj, half_lo(vv[t][e]), acc[2 * e]);
                acc[2 * e + 1] = fmaf(pj, half_hi(vv[t][e]), acc[2 * e + 1]);
            }
        }
    }
    if (ks < rpp)
#pragma unroll
        for (int e = 0; e < 8; ++e)
            part[ks * dg + kl * 8 + e] = acc[e]; // rpp * dg <= 256 * 8
    __syncthreads();
    if (tid < dg)
    {
        float o = 0.f;
        for (uint32_t k = 0; k < rpp; ++k)
            o += part[k * dg + tid];
        out[tid] = f2h(o);
    }
}

// Short-context decode attention in one kernel: block (h, g) (the pv kernel's mapping) scores all kv keys of head h
// itself, reduces the softmax statistics within the block and forms the probability-weighted sum for its dim
// group. The G blocks of a head read the head's keys from one XCD's L2, so HBM sees them once; at long contexts
// that re-reading costs more than the two-kernel path, which the host switches to. LDS: kv floats.
__global__ __launch_bounds__(256) void attn_decode_small_kernel(AttnDecodeArgs a)
{
    extern __shared__ float sm[];
    __shared__ float rmax[4], rsum[4];
    __shared__ float part[2048];
    uint32_t h, g;
    attn_block_head(blockIdx.x, a.groups, h, g);
    if (h >= a.H)
        return;
    const uint32_t tid = threadIdx.x;
    const uint32_t kv = a.step->offset + 1;
    const uint16_t *Vh = a.vc + (size_t)h * a.ctx * a.hd;
    const uint32_t dg = a.hd / a.groups, d0 = g * dg;
    const uint32_t lpr = dg / 8, vpr = a.hd / 8, rpp = 256 / lpr;
    const uint32_t kl = tid % lpr, ks = tid / lpr;
    // this block's first V rows, in flight while the scores are computed
    constexpr int U = 8;
    const u32x4 *Vv = (const u32x4 *)Vh + d0 / 8 + kl;
    u32x4 vv[U];
#pragma unroll
    for (int t = 0; t < U; ++t)
        vv[t] = Vv[(size_t)min(ks + rpp * t, kv - 1) * vpr];
    attn_score_keys<16>(a.q + (size_t)h * a.hd, a.kc + (size_t)h * a.ctx * a.hd, kv, a.hd, a.scale, sm);
    __syncthreads();
    float mx = -FLT_MAX;
    for (uint32_t j = tid; j < kv; j += 256)
        mx = fmaxf(mx, sm[j]);
    const float M = block4_max(mx, rmax);
    float sum = 0.f;
    for (uint32_t j = tid; j < kv; j += 256)
        sum += expf(sm[j] - M);
    const float L = block4_sum(sum, rsum);
    for (uint32_t j = tid; j < kv; j += 256)
        sm[j] = h2f(f2h(expf(sm[j] - M) / L));
    __syncthreads();
    uint16_t *out = a.out + (size_t)h * a.hd + d0;
    if (kv == a.hd)
    {
        attn_pv_transposed(sm, Vh, out, kv, a.hd, d0, dg);
        return;
    }
    float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    for (uint32_t jb = ks; jb < kv; jb += rpp * U)
    {
        if (jb != ks)
        {
#pragma unroll
            for (int t = 0; t < U; ++t)
                vv[t] = Vv[(size_t)min(jb + rpp * t, kv - 1) * vpr];
        }
#pragma unroll
        for (int t = 0; t < U; ++t)
        {
            const uint32_t j = jb + rpp * t;
            const float pj = j < kv ? sm[min(j, kv - 1)] : 0.f;
#pragma unroll
            for (int e = 0; e < 4; ++e)
            {
                acc[2 * e] = fmaf(pj, half_lo(vv[t][e]), acc[2 * e]);
                acc[2 * e + 1] = fmaf(pj, half_hi(vv[t][e]), acc[2 * e + 1]);
            }
        }
    }
    if (ks < rpp)
#pragma unroll
        for (int e = 0; e < 8; ++e)
            part[ks * dg + kl * 8 + e] = acc[e];
    __syncthreads();
    if (tid < dg)
    {
        float o = 0.f;
        for (uint32_t k = 0; k < rpp; ++k)
            o += part[k * dg + tid];
        out[tid] = f2h(o);
    }
}

hipError_t launch_attn_small(hipStream_t st, const AttnDecodeArgs &a, uint32_t kv_max)
{
    if (a.hd % 8 != 0 || a.hd > 256 || a.H == 0 || a.groups == 0 || (a.hd / 8) % a.groups != 0 || kv_max == 0)
        return hipErrorInvalidValue;
    const uint32_t blocks = (a.H + 7) / 8 * 8 * a.groups;
    attn_decode_small_kernel<<<blocks, 256, (size_t)kv_max * sizeof(float), st>>>(a);
    return hipGetLastError();
}

static size_t attn_scores_lds(uint32_t hd, uint32_t ctx, uint32_t cmax)
{
    uint32_t ch = (ctx + cmax - 1) / cmax;
    ch = (ch + 15) / 16 * 16;
    return (size_t)(ch > hd ? ch : hd) * sizeof(float);
}

uint32_t attn_pv_groups(uint32_t H, uint32_t hd)
{
    // the largest divisor of the row's 16-byte vectors that is <= 8 while H * G stays <= 512 workgroups
    uint32_t best = 1;
    for (uint32_t g = 1; g <= 8; ++g)
        if ((hd / 8) % g == 0 && H * g <= 512)
            best = g;
    return best;
}

static bool attn_decode_ok(const AttnDecodeArgs &a)
{
    return a.hd % 8 == 0 && a.hd <= 256 && a.cmax > 0 && a.H > 0 && a.groups > 0 && (a.hd / 8) % a.groups == 0;
}

hipError_t launch_attn_scores(hipStream_t st, const AttnDecodeArgs &a)
{
    if (!attn_decode_ok(a))
        return hipErrorInvalidValue;
    attn_scores_kernel<<<a.H * a.cmax, 256, attn_scores_lds(a.hd, a.ctx, a.cmax), st>>>(a);
    return hipGetLastError();
}

hipError_t launch_attn_pv(hipStream_t st, const AttnDecodeArgs &a)
{
    if (!attn_decode_ok(a))
        return hipErrorInvalidValue;
    const uint32_t blocks = (a.H + 7) / 8 * 8 * a.groups;
    attn_pv_kernel<<<blocks, 256, 0, st>>>(a);
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
// ARG_MAX for contiguous fp16 rows, one pass: 16-byte loads, then wave shuffles and one LDS step under the
// reference's arg-max order (am_before), which is a total order, so the reduction tree does not matter.
__global__ __launch_bounds__(1024) void argmax_rows_kernel(const uint16_t *logits, uint32_t *ids, uint32_t V,
                                                           DecodeIo *io)
{
    __shared__ float wv[16];
    __shared__ uint32_t wi[16];
    const uint32_t t = threadIdx.x;
    const uint16_t *row = logits + (size_t)blockIdx.x * V;
    // threads without an element hold (-inf, ~0u), which every element precedes
    float bv = -INFINITY;
    uint32_t bi = 0xFFFFFFFFu;
    if ((V & 7u) == 0)
    {
        const u32x4 *rv = (const u32x4 *)row;
        const uint32_t nv = V / 8;
        for (uint32_t v0 = t; v0 < nv; v0 += 4 * 1024)
        {
            u32x4 xs[4];
#pragma unroll
            for (int k = 0; k < 4; ++k)
                xs[k] = rv[min(v0 + 1024 * k, nv - 1)]; // clamped unconditional loads, duplicates skipped below
#pragma unroll
            for (int k = 0; k < 4; ++k)
            {
                const uint32_t vi = v0 + 1024 * k;
                if (vi >= nv)
                    break;
                const u32x4 x = xs[k];
#pragma unroll
            for (int e = 0; e < 4; ++e)
            {
                const uint32_t i = vi * 8 + 2 * e;
                const float lo = half_lo(x[e]), hi = half_hi(x[e]);
                if (am_before(lo, i, bv, bi))
                {
                    bv = lo;
                    bi = i;
                }
                if (am_before(hi, i + 1, bv, bi))
                {
                    bv = hi;
                    bi = i + 1;
                }
            }
            }
        }
    }
    else
    {
        for (uint32_t i = t; i < V; i += 1024)
        {
            const float v = h2f(row[i]);
            if (am_before(v, i, bv, bi))
            {
                bv = v;
                bi = i;
            }
        }
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1)
    {
        const float v = __shfl_xor(bv, o, kWave);
        const uint32_t i = (uint32_t)__shfl_xor((int)bi, o, kWave);
        if (am_before(v, i, bv, bi))
        {
            bv = v;
            bi = i;
        }
    }
    if ((t & 63) == 0)
    {
        wv[t >> 6] = bv;
        wi[t >> 6] = bi;
    }
    __syncthreads();
    if (t == 0)
    {
        for (int w = 1; w < 16; ++w)
            if (am_before(wv[w], wi[w], bv, bi))
            {
                bv = wv[w];
                bi = wi[w];
            }
        ids[blockIdx.x] = bi;
        if (io && blockIdx.x == 0)
            io->id = bi;
    }
}

hipError_t launch_argmax_rows(hipStream_t st, const uint16_t *logits, uint32_t *ids, uint32_t S, uint32_t V,
                              DecodeIo *io)
{
    if (S == 0 || V == 0)
        return hipErrorInvalidValue;
    argmax_rows_kernel<<<S, 1024, 0, st>>>(logits, ids, V, io);
    return hipGetLastError();
}

} // namespace vk
