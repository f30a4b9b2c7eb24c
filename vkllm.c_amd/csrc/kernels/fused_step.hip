// Fused gfx950 kernels of the LLaMA-2 token step (src/models/vkllm_llama2_layers.c:13-354 as fused stages).
//
// Every stage rounds to fp16 exactly where the reference's graph materialises an fp16 tensor (norm output,
// Q/K/V, RoPE output, scores, probabilities, attention output, projection outputs, residual sums, SiLU(gate),
// up*gate, logits), so fusing changes only fp32 summation order.
//
// Decode (one token) runs five kernels per layer (six beyond the one-kernel attention's cache length):
//   gemv<QKV>      RMSNorm prologue, [Wq;Wk;Wv] rows, RoPE on q/k, k/v appended to the caches
//   attention      short caches: one kernel per step (attn_decode_small); long caches: attn_scores (scores and
//                  per-chunk softmax statistics) then attn_pv (probabilities with the row's statistics, P.V per
//                  chunk, chunk merge by the last block)
//   gemv<RESID>    Wo rows, residual add in place
//   gemv<GATEUP>   RMSNorm prologue, up and gate rows side by side, SiLU(gate)*up
//   gemv<RESID>    Wd rows, residual add in place
#include <float.h>

#include "attn_common.h"
#include "device_common.h"
#include "gemv_common.h"
#include "kernels.h"

namespace vk
{

// ---------------------------------------------------------------------------------------------------------------
// EMBEDDING (src/shaders/vkllm_embedding.comp:41-70) for contiguous rows
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
                                    uint32_t D, uint32_t unk, const uint32_t *prev_id)
{
    const uint32_t offset = io->offset;
    uint32_t tok = io->token_dev ? *prev_id : io->token;
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
                               uint32_t V, uint32_t D, uint32_t unk, const uint32_t *prev_id)
{
    if (D % 8 != 0 || !prev_id)
        return hipErrorInvalidValue;
    embed_decode_kernel<<<1, 256, 0, st>>>(io, step, embd, h, V, D, unk, prev_id);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------------------------------------------
// RMSNORM (src/shaders/vkllm_rmsnorm.comp:31-82): y = fp16((x * w) * (1 / sqrt(sum(x^2) / D + eps)))

// 512 threads a row, the block size of the norm fused into the residual products' split-K reduce (same sum order)
__global__ __launch_bounds__(512) void rmsnorm_rows_kernel(const uint16_t *x, const float *w, uint16_t *y, uint32_t D,
                                                           float eps, bool xt)
{
    __shared__ float red[8];
    const size_t s = blockIdx.x;
    if (xt)
        rmsnorm_row_to(x + s * D, w, (u32x4 *)y, D, eps, red, (int)s);
    else
        rmsnorm_row_to(x + s * D, w, (u32x4 *)(y + s * D), D, eps, red);
}

hipError_t launch_rmsnorm_rows(hipStream_t st, const uint16_t *x, const float *w, uint16_t *y, uint32_t S,
                               uint32_t D, float eps, bool xt)
{
    if (xt && (S > 128 || D % 16 != 0))
        return hipErrorInvalidValue;
    rmsnorm_rows_kernel<<<S, 512, 0, st>>>(x, w, y, D, eps, xt);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------------------------------------------
// GEMV: one wave per work unit (two weight rows), each lane streaming 16-byte slices of both rows against the
// input vector held in LDS, fp32 accumulation with widening FMAs, DPP wave reduction. Workgroups of four waves
// walk the units grid-stride so the prologue (input vector, optional RMSNorm) is paid once per workgroup.
constexpr int kGemvUnroll = 8;

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
    case EPI_RAW: // the plain kernel normalises only when norm_w is given
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

// the QKV product's epilogues (RoPE on q, k; k and v appended to the caches)
constexpr bool is_qkv(int epi)
{
    return epi == EPI_QKV || epi == EPI_QKV_ATTN;
}

// GEMV with the input prologue overlapped by the weight stream. A wave owns units of R weight rows (R/2 up rows
// next to R/2 gate rows for EPI_GATEUP; R even for EPI_QKV so RoPE pairs stay together); lane l holds the 16-byte
// vectors l + 64 i (i < NV) of each row, so NV * 512 >= K. Order of work in a workgroup:
//   1. its threads' share of the input vector (and of the RMSNorm weights) into registers
//   2. the weight vectors of each wave's first unit: the bulk of the traffic is in flight from here on
//   3. RMSNorm over the registers (block reduction in LDS), the normalised input into LDS
//   4. per unit: dot products against LDS, the next unit's weights issued before this unit's reduction
// Vector-memory counters retire in issue order, so waiting for the input (issued first) never waits for weights.
// EPI_QKV_ATTN then finishes each head's attention in the workgroup that completes the head's rows.
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

// Inputs of the epilogue are fetched with the unit's weights: EPI_QKV fq[k / 2], the RoPE denominator of pair
// (rows[k], rows[k + 1]); EPI_RESID rs[k], the residual at rows[k].
template <int EPI, int R> __device__ __forceinline__ void gemv_epilogue(const GemvArgs &a, uint32_t u,
                                                                        const uint32_t *rows, const float *acc,
                                                                        const float *fq, const float *rs)
{
    if (EPI == EPI_PLAIN || EPI == EPI_ARGMAX || EPI == EPI_RAW)
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
                a.out[rows[k]] = f2h(rs[k] + h2f(f2h(acc[k])));
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
            if constexpr (EPI == EPI_QKV_ATTN)
            {
                // the pair as one agent-scope store, written through to where another XCD's workgroup reads it
                if (region == 2)
                {
                    store_pair<true>(a.vc + cache, v0, v1);
                    continue;
                }
                const float f = (float)pos / fq[k / 2];
                const float c = cosf(f), sn = sinf(f);
                store_pair<true>(region == 0 ? a.out + rr : a.kc + cache, rope_mul_sub(c, v0, sn, v1),
                                 rope_mul_add(sn, v0, c, v1));
                continue;
            }
            if (region == 2)
            {
                a.vc[cache] = f2h(v0);
                a.vc[cache + 1] = f2h(v1);
                continue;
            }
            const float f = (float)pos / fq[k / 2];
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

// the epilogues whose input is the RMSNorm of the residual stream (all but the residual products)
constexpr bool gemv_normalises(int epi)
{
    return epi != EPI_RESID && epi != EPI_RAW;
}

// EPI_QKV_ATTN's tail, all 256 threads of the workgroup: single-token attention of head `head` over kv positions
// (src/models/vkllm_llama2_layers.c:223-257 with src/shaders/vkllm_softmax.comp:42-96), with the reference's rounding
// points: s_j = fp16(scale q.k_j) (the key layout and sums of the short-cache kernel), M and L over all kv scores,
// p_j = fp16(exp(s_j - M) / L), out[d] = fp16(sum_j p_j v_j[d]); kv == hd takes the transposed product p . V^T.
// sm (the input row's LDS, sized for this) holds kAttnTailMaxKv scores followed by 4 * hd partial sums. The caller has acquired the head's rows (q and this
// position's K and V rows were stored by other workgroups of this launch).
__device__ void qkv_attention_tail(const GemvArgs &a, uint32_t head, float *sm)
{
    constexpr uint32_t NT = 256, NW = NT / 64;
    constexpr int U = 8, UV = 8;
    const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint32_t hd = a.hd, kv = a.step->offset + 1, vpr = hd / 8;
    const uint16_t *Kh = a.kc + (size_t)head * a.ctx * hd, *Vh = a.vc + (size_t)head * a.ctx * hd;
    uint16_t *out = a.attn_out + (size_t)head * hd;
    // V rows: lane = (vector vl, row slot within the wave); the block covers `slots` rows per pass, the first UV
    // passes requested before the scores
    const uint32_t seg = 64 / vpr, vl = lane / seg, rs = wave * seg + lane % seg, slots = NW * seg;
    const u32x4 *Vv = (const u32x4 *)Vh + vl;
    const bool transposed = kv == hd;
    u32x4 vv[UV];
#pragma unroll
    for (int t = 0; t < UV; ++t)
        vv[t] = Vv[(size_t)min(rs + slots * t, kv - 1) * vpr];
    const KeyLayout k = key_layout<NT>(a.out + (size_t)head * hd, hd);
    const u32x4 *Kv = (const u32x4 *)Kh;
    for (uint32_t jb = k.ks; jb < kv; jb += k.kpp * U)
    {
        u32x4 ka[U], kb[U];
        load_keys<U>(k, Kv, jb, kv - 1, ka, kb);
        score_keys<U>(k, ka, kb, jb, kv, a.attn_scale, sm);
    }
    __syncthreads();
    // softmax statistics, reduced by every wave over all kv scores
    float M = -FLT_MAX;
    for (uint32_t j = lane; j < kv; j += 64)
        M = fmaxf(M, sm[j]);
    M = wave_max_dpp(M);
    float L = 0.f;
    for (uint32_t j = lane; j < kv; j += 64)
        L += expf(sm[j] - M);
    L = wave_sum_dpp(L);
    if (transposed)
    {
        __syncthreads(); // every wave has its statistics before the scores become probabilities
        for (uint32_t j = tid; j < kv; j += NT)
            sm[j] = h2f(f2h(expf(sm[j] - M) / L));
        __syncthreads();
        for (uint32_t r = 2 * tid; r < hd; r += 2 * NT)
        {
            const uint16_t *row0 = Vh + (size_t)r * hd, *row1 = row0 + hd;
            float a0 = 0.f, a1 = 0.f;
            for (uint32_t j = 0; j < kv; ++j)
            {
                a0 = fmaf(sm[j], h2f(row0[j]), a0);
                a1 = fmaf(sm[j], h2f(row1[j]), a1);
            }
            store_pair<false>(out + r, a0, a1);
        }
        __syncthreads();
        return;
    }
    float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    const uint32_t passes = (kv + slots - 1) / slots;
    for (uint32_t t0 = 0; t0 < passes; t0 += UV)
    {
        if (t0 > 0) // the next UV passes of V rows, all requested at once
#pragma unroll
            for (int t = 0; t < UV; ++t)
                vv[t] = Vv[(size_t)min(rs + slots * (t0 + t), kv - 1) * vpr];
#pragma unroll
        for (int t = 0; t < UV; ++t)
        {
            const uint32_t j = rs + slots * (t0 + t);
            const bool live = j < kv;
            const float pj = live ? h2f(f2h(expf(sm[min(j, kv - 1)] - M) / L)) : 0.f;
#pragma unroll
            for (int e = 0; e < 4; ++e)
            {
                const uint32_t w = live ? vv[t][e] : 0u;
                acc[2 * e] = fmaf(pj, half_lo(w), acc[2 * e]);
                acc[2 * e + 1] = fmaf(pj, half_hi(w), acc[2 * e + 1]);
            }
        }
    }
    float *part = sm + kAttnTailMaxKv; // NW rows of hd partial sums
#pragma unroll
    for (int e = 0; e < 8; ++e)
        acc[e] = group_sum(acc[e], seg);
    if (lane % seg == 0)
#pragma unroll
        for (int e = 0; e < 8; ++e)
            part[wave * hd + vl * 8 + e] = acc[e];
    __syncthreads();
    if (2 * tid < hd)
    {
        float o0 = 0.f, o1 = 0.f;
#pragma unroll
        for (uint32_t w = 0; w < NW; ++w)
        {
            o0 += part[w * hd + 2 * tid];
            o1 += part[w * hd + 2 * tid + 1];
        }
        store_pair<false>(out + 2 * tid, o0, o1);
    }
    __syncthreads();
}

// EPI_QKV_ATTN after the workgroup's last unit: each head's completed units are counted (the wave's stores are
// agent-scope and complete first, the same hand-off as the vocabulary product's arg max), and the workgroup whose
// count completes a head computes that head's attention. No workgroup waits for another.
template <int R>
__device__ __forceinline__ void qkv_attention_heads(const GemvArgs &a, uint32_t *head_done, float *sm)
{
    __shared__ uint32_t todo[kAttnTailMaxHeads];
    __shared__ uint32_t ntodo;
    const uint32_t tid = threadIdx.x;
    const uint32_t per_head = 3 * a.hd / R; // units holding a head's q, k and v rows
    __builtin_amdgcn_s_waitcnt(0);
    if (tid == 0)
        ntodo = 0;
    __syncthreads();
    if (tid < a.H && head_done[tid] != 0)
    {
        const uint32_t n = head_done[tid];
        if (__hip_atomic_fetch_add(a.head_count + tid, n, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) + n == per_head)
            todo[atomicAdd(&ntodo, 1u)] = tid;
    }
    __syncthreads();
    const uint32_t n = ntodo;
    if (n == 0)
        return;
    if (a.step->offset + 1 > kAttnTailMaxKv)
    {
        // a position past what the launch was chosen for (the host picks the kernel by position): flag the step
        if (tid == 0 && a.attn_err)
            __hip_atomic_store(a.attn_err, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
        for (uint32_t i = 0; i < n && tid == 0; ++i)
            __hip_atomic_store(a.head_count + todo[i], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        return;
    }
    // the completing workgroup acquires what the head's other workgroups stored
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
    for (uint32_t i = 0; i < n; ++i)
    {
        const uint32_t head = todo[i];
        qkv_attention_tail(a, head, sm);
        if (tid == 0)
            __hip_atomic_store(a.head_count + head, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}

template <int EPI, int R, int NV> __global__ __launch_bounds__(256) void gemv_fast_kernel(GemvArgs a, uint32_t units)
{
    extern __shared__ u32x4 xs[];
    __shared__ float red[8];
    constexpr int XV = (NV * 64 + 255) / 256; // input vectors per thread
    const uint32_t tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
    const uint32_t nvec = a.K / 8;
    // the residual products (Wo, Wd) take their input as is; the others normalise it (the launcher checks norm_w)
    constexpr bool norm = gemv_normalises(EPI);

    // EPI_QKV_ATTN: units completed per head by this workgroup
    __shared__ uint32_t head_done[EPI == EPI_QKV_ATTN ? kAttnTailMaxHeads : 1];
    if constexpr (EPI == EPI_QKV_ATTN)
        if (tid < kAttnTailMaxHeads)
            head_done[tid] = 0;

    // 1. input share (and RMSNorm weights)
    // Loads are unconditional at clamped addresses (a guarded load compiles to a branch and a full wait per load);
    // lanes past the end read a valid duplicate that is masked out below.
    u32x4 xr[XV];
    float4 nw[norm ? XV : 1][2];
    const float4 *nwp = (const float4 *)(norm ? a.norm_w : (const float *)a.x);
#pragma unroll
    for (int i = 0; i < XV; ++i)
    {
        const uint32_t vi = min(tid + 256 * i, nvec - 1);
        xr[i] = ((const u32x4 *)a.x)[vi];
        if constexpr (norm)
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
    // the epilogue's inputs (RoPE denominators, residuals), requested ahead of the unit's weights: a request in the
    // epilogue would wait for the next unit's weights, as counters retire in issue order
    constexpr int NF = is_qkv(EPI) && R >= 2 ? R / 2 : 1, NR = EPI == EPI_RESID ? R : 1;
    float fq[NF], rs[NR];
#pragma unroll
    for (int k = 0; k < NF; ++k)
        fq[k] = 1.f;
#pragma unroll
    for (int k = 0; k < NR; ++k)
        rs[k] = 0.f;
    auto load_unit = [&](uint32_t unit) {
        gemv_rows_of<EPI>(a, unit, R, rows);
        if (is_qkv(EPI))
#pragma unroll
            for (int k = 0; k < NF; ++k)
                fq[k] = a.freqs[((unit < units && rows[2 * k] < a.rows ? rows[2 * k] : 0) % a.D) % a.hd / 2];
        if (EPI == EPI_RESID)
#pragma unroll
            for (int k = 0; k < NR; ++k)
                rs[k] = h2f(a.resid[unit < units && rows[k] < a.rows ? rows[k] : 0]);
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
    if constexpr (norm)
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

    // 4. units (EPI_ARGMAX: lane 0 keeps the best of the rows it stores)
    float bv = -INFINITY;
    uint32_t bi = 0xFFFFFFFFu;
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
        float cur_fq[NF], cur_rs[NR];
#pragma unroll
        for (int k = 0; k < R; ++k)
            cur_rows[k] = rows[k];
#pragma unroll
        for (int k = 0; k < NF; ++k)
            cur_fq[k] = fq[k];
#pragma unroll
        for (int k = 0; k < NR; ++k)
            cur_rs[k] = rs[k];
        const uint32_t cur = u;
        u += stride;
        if (u < units)
            load_unit(u);
#pragma unroll
        for (int k = 0; k < R; ++k)
            acc[k] = wave_sum_dpp(acc[k]);
        if (lane == 0)
        {
            gemv_epilogue<EPI, R>(a, cur, cur_rows, acc, cur_fq, cur_rs);
            if constexpr (EPI == EPI_QKV_ATTN)
                atomicAdd(&head_done[(cur_rows[0] % a.D) / a.hd], 1u);
            if constexpr (EPI == EPI_ARGMAX)
#pragma unroll
                for (int k = 0; k < R; ++k)
                {
                    const float v = h2f(f2h(acc[k]));
                    if (cur_rows[k] < a.rows && am_before(v, cur_rows[k], bv, bi))
                    {
                        bv = v;
                        bi = cur_rows[k];
                    }
                }
        }
    }
    if constexpr (EPI == EPI_ARGMAX)
        gemv_argmax_finish(a, bv, bi);
    if constexpr (EPI == EPI_QKV_ATTN)
        qkv_attention_heads<R>(a, head_done, (float *)xs);
}

// Residual GEMV over long rows (K > 8192: the down product, K = FFN width): a workgroup per unit of R rows, its 4
// waves splitting each row's 16-byte vectors (wave w, lane l: vectors 64 w + l + 256 i, i < NVW). A wave streaming a
// whole 22 KB row by itself reads at 5.4 TB/s on this GPU; spread over the workgroup the same bytes stream at
// 6.8-6.9 TB/s. The workgroup takes units blockIdx.x + n gridDim.x (n < kWgMaxUnits); each wave reduces its partial
// sums per unit into LDS without waiting for the others (the next unit's weights are requested before the
// reduction), and after the last unit thread t finishes row t: out[r] = fp16(resid[r] + fp16(sum)), the four wave
// partials added in wave order, the residual requested when the kernel starts.
constexpr uint32_t kWgMaxUnits = 8;
template <int R, int NVW> __global__ __launch_bounds__(256) void gemv_wg_resid_kernel(GemvArgs a, uint32_t units)
{
    extern __shared__ u32x4 xs[];
    __shared__ float part[kWgMaxUnits][4][R];
    const uint32_t tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
    const uint32_t nvec = a.K / 8;
    // 1. the input row (loads unconditional at clamped addresses; lanes past the end are zeroed below), and the
    // residual of the row this thread finishes
    u32x4 xr[NVW];
#pragma unroll
    for (int i = 0; i < NVW; ++i)
        xr[i] = ((const u32x4 *)a.x)[min(tid + 256 * i, nvec - 1)];
    const uint32_t my_unit = blockIdx.x + (tid / R) * gridDim.x, my_row = my_unit * R + tid % R;
    const bool finisher = tid < kWgMaxUnits * R && my_unit < units && my_row < a.rows;
    const float my_rs = h2f(a.resid[finisher ? my_row : 0]);
    // 2. the first unit's weights
    u32x4 w[R][NVW];
    auto load_unit = [&](uint32_t unit) {
#pragma unroll
        for (int k = 0; k < R; ++k)
        {
            const u32x4 *wr = (const u32x4 *)(a.w + (size_t)min(unit * R + k, a.rows - 1) * a.K);
#pragma unroll
            for (int i = 0; i < NVW; ++i)
                w[k][i] = __builtin_nontemporal_load(wr + min(tid + 256 * i, nvec - 1));
        }
    };
    uint32_t u = blockIdx.x;
    if (u < units)
        load_unit(u);
#pragma unroll
    for (int i = 0; i < NVW; ++i)
    {
        const uint32_t vi = tid + 256 * i;
        if (vi < nvec)
            xs[vi] = xr[i];
    }
    __syncthreads();
    // 3. units
    for (uint32_t n = 0; u < units; u += gridDim.x, ++n)
    {
        float acc[R];
#pragma unroll
        for (int k = 0; k < R; ++k)
            acc[k] = 0.f;
#pragma unroll
        for (int i = 0; i < NVW; ++i)
        {
            const uint32_t vi = tid + 256 * i;
            if (vi < nvec)
            {
                const u32x4 xv = xs[vi];
#pragma unroll
                for (int k = 0; k < R; ++k)
                    acc[k] = dot8(w[k][i], xv, acc[k]);
            }
        }
        if (u + gridDim.x < units)
            load_unit(u + gridDim.x);
#pragma unroll
        for (int k = 0; k < R; ++k)
            acc[k] = wave_sum_dpp(acc[k]);
        if (lane == 0)
#pragma unroll
            for (int k = 0; k < R; ++k)
                part[n][wid][k] = acc[k];
    }
    __syncthreads();
    // 4. the rows
    if (finisher)
    {
        const uint32_t n = tid / R, k = tid % R;
        const float sum = ((part[n][0][k] + part[n][1][k]) + part[n][2][k]) + part[n][3][k];
        a.out[my_row] = f2h(my_rs + h2f(f2h(sum)));
    }
}

template <int R, int NVW> static hipError_t launch_wg_resid(hipStream_t st, const GemvArgs &a, int cu_count)
{
    const uint32_t units = (a.rows + R - 1) / R;
    const size_t lds = (size_t)a.K * 2;
    static uint64_t occ_memo = 0;
    const int per_cu = std::max(occupancy_per_cu((const void *)gemv_wg_resid_kernel<R, NVW>, 256, lds, occ_memo), 1);
    // two workgroups per CU (1, 2 and 3 measure within 2% of each other for the 7B down product), and at most
    // kWgMaxUnits units per workgroup
    const uint32_t cap = (uint32_t)(cu_count > 0 ? cu_count : 256) * (uint32_t)std::min(per_cu, 2);
    const uint32_t grid = std::max(std::min(units, cap), (units + kWgMaxUnits - 1) / kWgMaxUnits);
    gemv_wg_resid_kernel<R, NVW><<<grid, 256, lds, st>>>(a, units);
    return hipGetLastError();
}

// units of R rows for `a`; 0 when R does not fit the epilogue's pairing
static uint32_t gemv_units(int epi, const GemvArgs &a, int R)
{
    if (epi == EPI_GATEUP)
        return (R % 2 == 0 && a.rows % R == 0) ? a.rows / R : 0;
    if (is_qkv(epi) && R % 2 != 0)
        return 0;
    return (a.rows + R - 1) / R;
}

template <int EPI, int R, int NV> static hipError_t launch_fast(hipStream_t st, const GemvArgs &a, int cu_count)
{
    const uint32_t units = gemv_units(EPI, a, R);
    if (units == 0 || (a.norm_w != nullptr) != gemv_normalises(EPI))
        return hipErrorInvalidValue;
    // resident workgroups per CU at this kernel's register use and this K's LDS (at least 1: it only sizes the grid)
    static uint64_t occ_memo = 0;
    // the input row (EPI_QKV_ATTN: at least the attention tail's scores and partial sums)
    const size_t lds = EPI == EPI_QKV_ATTN ? std::max((size_t)a.K * 2, (kAttnTailMaxKv + 4 * a.hd) * sizeof(float))
                                           : (size_t)a.K * 2;
    const int per_cu = std::max(occupancy_per_cu((const void *)gemv_fast_kernel<EPI, R, NV>, 256, lds, occ_memo), 1);
    // every wave gets the same number of units (the fewest that the resident waves can cover), so no wave runs an
    // extra unit while the others idle. Kernels of at most 4 resident workgroups per CU (two rows per unit, or long
    // rows) run 2 per CU: fewer, longer-lived waves stream as many bytes with less start-up per wave (7B widths:
    // QKV 768 -> 512 workgroups 18.9 -> 18.3 us, gate/up 688 -> 459 29.4 -> 28.9 us, logits 1000 -> 500 40.9 ->
    // 40.4 us; Wo, 7 per CU, is fastest at one unit per wave)
    const uint32_t resident = per_cu <= 4 ? (uint32_t)std::min(per_cu, 2) : (uint32_t)per_cu;
    const uint32_t cap = (uint32_t)(cu_count > 0 ? cu_count : 256) * resident;
    const uint32_t per_wave = (units + 4 * cap - 1) / (4 * cap);
    const uint32_t blocks = (units + 4 * per_wave - 1) / (4 * per_wave);
    if (EPI == EPI_ARGMAX && (blocks > a.am_cap || !a.am_ids || !a.am_val || !a.am_idx || !a.am_count))
        return hipErrorInvalidValue;
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
// EPI_ARGMAX: one row per unit (the vocabulary product)
static hipError_t launch_argmax_epi(hipStream_t st, const GemvArgs &a, int cu_count, int NV)
{
    constexpr int EPI = EPI_ARGMAX;
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
    return hipErrorInvalidValue;
}
#undef GEMV_NV_CASE

// rows per unit: the number of 16-byte vectors each lane keeps in flight is R * NV
static int gemv_default_r(int epi, uint32_t K)
{
    (void)K;
    return epi == EPI_GATEUP || is_qkv(epi) ? 2 : 1;
}

hipError_t launch_gemv(hipStream_t st, int epi, const GemvArgs &a, int cu_count)
{
    if (a.K % 8 != 0 || a.rows == 0)
        return hipErrorInvalidValue;
    const uint32_t nvec = a.K / 8;
    int R = a.rows_per_unit ? (int)a.rows_per_unit : gemv_default_r(epi, a.K);
    if (R == 1 && (epi == EPI_GATEUP || is_qkv(epi)))
        R = 2;
    // the attention tail: a head's V row as 4 to 64 16-byte vectors (a lane each)
    if (epi == EPI_QKV_ATTN && (R != 2 || a.H > kAttnTailMaxHeads || a.hd % 8 != 0 || a.hd < 32 ||
                                64 % (a.hd / 8) != 0 || !a.head_count || !a.attn_out))
        return hipErrorInvalidValue;
    // long rows of the residual product: split over the workgroup's waves (unless a unit size is asked for)
    if (epi == EPI_RESID && !a.rows_per_unit && nvec > 1024 && nvec <= 2048 && a.resid && a.out)
        switch ((nvec + 255) / 256)
        {
        case 5:
            return launch_wg_resid<2, 5>(st, a, cu_count);
        case 6:
            return launch_wg_resid<2, 6>(st, a, cu_count);
        case 7:
            return launch_wg_resid<2, 7>(st, a, cu_count);
        case 8:
            return launch_wg_resid<2, 8>(st, a, cu_count);
        }
    const int NV = (R == 1 || R == 2 || R == 4) ? gemv_pick_nv(R, nvec) : 0;
    if (NV != 0 && (epi != EPI_GATEUP || a.rows % R == 0))
    {
        switch (epi)
        {
        case EPI_PLAIN:
            return launch_epi<EPI_PLAIN>(st, a, cu_count, R, NV);
        case EPI_RAW:
            return launch_epi<EPI_RAW>(st, a, cu_count, R, NV);
        case EPI_RESID:
            return launch_epi<EPI_RESID>(st, a, cu_count, R, NV);
        case EPI_GATEUP:
            return launch_epi<EPI_GATEUP>(st, a, cu_count, R, NV);
        case EPI_QKV:
            return launch_epi<EPI_QKV>(st, a, cu_count, R, NV);
        case EPI_QKV_ATTN:
            return launch_epi<EPI_QKV_ATTN>(st, a, cu_count, R, NV);
        case EPI_ARGMAX:
            return R == 1 ? launch_argmax_epi(st, a, cu_count, NV) : hipErrorInvalidValue;
        default:
            return hipErrorInvalidValue;
        }
    }
    return epi == EPI_ARGMAX || epi == EPI_QKV_ATTN ? hipErrorInvalidValue : launch_gemv_loop(st, epi, a, cu_count);
}

// ---------------------------------------------------------------------------------------------------------------
// Attention for one query row of one head (src/models/vkllm_llama2_layers.c:223-257 with
// src/shaders/vkllm_softmax.comp:42-96): s_j = fp16(scale * q.k_j), j < kv; max over all kv scores (the softmax
// shader's row max includes the masked positions); sum and p = fp16(exp(s - max) / sum) over j < causal, p = 0
// beyond; out[d] = fp16(sum_j p_j V[j][d]) for d in [d0, d0 + dn); with `transposed`, out[n] = fp16(sum_k p_k
// V[n][k]). `sm` holds kv floats. All 256 threads of the block take part.
__device__ void attn_row(const uint16_t *q, const uint16_t *K, const uint16_t *V, uint16_t *out, uint32_t kv,
                         uint32_t causal, uint32_t hd, float scale, bool transposed, uint32_t d0, uint32_t dn,
                         float *sm, float *red, float *part)
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
    for (uint32_t j = tid; j < causal; j += 256)
        sum += expf(sm[j] - mx);
    sum = block_sum(sum, red);
    for (uint32_t j = tid; j < kv; j += 256)
        sm[j] = j < causal ? h2f(f2h(expf(sm[j] - mx) / sum)) : 0.f;
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

// prefill for head sizes without an MFMA kernel: one workgroup per (query row, head); the transposition rule
// applies when the step's kv == hd
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
             offset + S, offset + s + 1, hd, scale, transposed, 0, hd, sm, red, part);
}

hipError_t launch_attn_prefill(hipStream_t st, const uint16_t *q, const uint16_t *kc, const uint16_t *vc,
                               uint16_t *out, uint32_t offset, uint32_t S, uint32_t H, uint32_t hd, uint32_t ctx,
                               float scale, bool xt)
{
    if (hd % 8 != 0 || hd > 256)
        return hipErrorInvalidValue;
    if (attn_prefill_mfma_ok(hd))
        return launch_attn_prefill_mfma(st, q, kc, vc, out, offset, S, H, hd, ctx, scale, xt);
    if (xt) // fragment-ordered output from the MFMA kernel only
        return hipErrorInvalidValue;
    const size_t lds = (size_t)(offset + S) * sizeof(float);
    attn_prefill_kernel<<<dim3(S, H), 256, lds, st>>>(q, kc, vc, out, offset, S, H, hd, ctx, scale);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------------------------------------------
// RoPE (normal style, src/shaders/vkllm_rope.comp:39-79) on q and k of a prefill QKV block, k and v appended to
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

// RoPE angles of a prompt step, once for all layers: the same f = pos / freqs[w] and cosf / sinf as rope_kv_kernel
__global__ void rope_table_kernel(float *cs, const float *freqs, uint32_t offset, uint32_t S, uint32_t half)
{
    const uint64_t total = (uint64_t)S * half;
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += (uint64_t)gridDim.x * blockDim.x)
    {
        const uint32_t s = (uint32_t)(i / half), w = (uint32_t)(i % half);
        const float f = (float)(offset + s) / freqs[w];
        cs[2 * i] = cosf(f);
        cs[2 * i + 1] = sinf(f);
    }
}

hipError_t launch_rope_table(hipStream_t st, float *cs, const float *freqs, uint32_t offset, uint32_t S, uint32_t hd)
{
    const uint64_t total = (uint64_t)S * (hd / 2);
    uint32_t grid = (uint32_t)((total + 255) / 256);
    grid = grid > 4096 ? 4096 : grid;
    rope_table_kernel<<<grid, 256, 0, st>>>(cs, freqs, offset, S, hd / 2);
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
    // threads without an element hold (-inf, ~0u), which every element precedes. In a row shorter than 32 the
    // reference's lanes l in [V, 32) enter its reduction with (-FLT_MAX, l) (src/shaders/vkllm_arg_max.comp:55-60),
    // which wins over a row of -inf: those lanes join here as elements of their own.
    float bv = -INFINITY;
    uint32_t bi = 0xFFFFFFFFu;
    if (t >= V && t < 32)
    {
        bv = -FLT_MAX;
        bi = t;
    }
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
