// Decode attention of the LLaMA-2 token step: one query row per head against the KV cache
// (src/models/vkllm_llama2_layers.c:223-257 with src/shaders/vkllm_softmax.comp:42-96 and
// src/shaders/vkllm_mat_mul_vec.comp:94-150 for the two products).
//
// The reference materialises fp16 scores, fp16 probabilities and an fp16 attention output, so each probability is
// rounded with the GLOBAL max and sum of its row. Both paths keep those rounding points:
//   short caches (one kernel, attn_decode_small_kernel): block (h, g) scores all kv keys of head h itself, reduces
//     the softmax statistics in the block and forms the probability-weighted sum for its slice of the head's dims.
//   long caches (two kernels over fixed chunks of `chunk` positions): attn_scores_kernel writes fp16-rounded
//     scores and each chunk's max and sum of exp; attn_pvc_kernel reduces those statistics (identically in every
//     block of the head), rounds the chunk's probabilities, forms its partial sums, and the last chunk block of a
//     head to finish adds the partials in chunk order.
// No kernel uses a device-wide fence (on this GPU one writes back a whole L2); kv == hd takes the reference's
// transposed product p . V^T.
#include <float.h>

#include "device_common.h"
#include "kernels.h"

namespace vk
{

// power of two >= n
__device__ __forceinline__ uint32_t lanes_pow2(uint32_t n)
{
    uint32_t l = 1;
    while (l < n)
        l <<= 1;
    return l;
}

// Lanes sharing one cache row when scoring keys: each lane takes two 16-byte vectors (16 dims) of the row.
__device__ __forceinline__ uint32_t key_lanes(uint32_t hd)
{
    uint32_t l = 1;
    while (l * 16 < hd)
        l <<= 1;
    return l;
}

// Scoring layout: lane kl of a key group holds dims [16 kl, 16 kl + 16) as vectors c0, c1 (clamped into the row;
// lanes past the row multiply a zero query).
struct KeyLayout
{
    uint32_t vpr, lpk, kl, ks, kpp, c0, c1;
    u32x4 q0, q1;
};

template <int NT> __device__ __forceinline__ KeyLayout key_layout(const uint16_t *q, uint32_t hd)
{
    KeyLayout k;
    k.vpr = hd / 8;
    k.lpk = key_lanes(hd);
    k.kl = threadIdx.x % k.lpk;
    k.ks = threadIdx.x / k.lpk;
    k.kpp = NT / k.lpk;
    k.c0 = min(2 * k.kl, k.vpr - 1);
    k.c1 = min(2 * k.kl + 1, k.vpr - 1);
    const u32x4 *qv = (const u32x4 *)q;
    k.q0 = qv[k.c0];
    k.q1 = qv[k.c1];
    if (2 * k.kl >= k.vpr)
        k.q0 = (u32x4){0, 0, 0, 0};
    if (2 * k.kl + 1 >= k.vpr)
        k.q1 = (u32x4){0, 0, 0, 0};
    return k;
}

// U passes of keys starting at key jb of this thread's group: rows min(jb + kpp t, last)
template <int U>
__device__ __forceinline__ void load_keys(const KeyLayout &k, const u32x4 *Kv, uint32_t jb, uint32_t last, u32x4 *ka,
                                          u32x4 *kb)
{
#pragma unroll
    for (int t = 0; t < U; ++t)
    {
        const size_t row = (size_t)min(jb + k.kpp * t, last) * k.vpr;
        ka[t] = Kv[row + k.c0];
        kb[t] = Kv[row + k.c1];
    }
}

// sm[j] = fp16(scale * q . K[j]) for the loaded keys j = jb + kpp t < n. The lanes of one key share jb, so the group
// DPP only combines live lanes.
template <int U>
__device__ __forceinline__ void score_keys(const KeyLayout &k, const u32x4 *ka, const u32x4 *kb, uint32_t jb,
                                           uint32_t n, float scale, float *sm)
{
#pragma unroll
    for (int t = 0; t < U; ++t)
    {
        float p = dot8(kb[t], k.q1, dot8(ka[t], k.q0, 0.f));
        p = group_sum(p, k.lpk);
        const uint32_t j = jb + k.kpp * t;
        if (k.kl == 0 && j < n)
            sm[j] = h2f(f2h(p * scale));
    }
}

// out[r] = fp16(sum_k p_k V[r][k]) for the block's rows r of the reference's transposed product (kv == hd)
__device__ __forceinline__ void pv_transposed(const float *pl, const uint16_t *Vh, uint16_t *out, uint32_t kv,
                                              uint32_t hd, uint32_t d0, uint32_t dg)
{
    for (uint32_t r = threadIdx.x; r < dg; r += blockDim.x)
    {
        const uint16_t *row = Vh + (size_t)(d0 + r) * hd;
        float acc = 0.f;
        for (uint32_t k = 0; k < kv; ++k)
            acc = fmaf(pl[k], h2f(row[k]), acc);
        out[r] = f2h(acc);
    }
}

// out[d] = fp16(sum over row groups of part[group][d]) for d < dg; `part` holds rpp rows of dg partial sums and is
// reused as scratch. Two stages keep every thread's chain short.
template <int NT> __device__ __forceinline__ void pv_reduce_out(float *part, uint32_t rpp, uint32_t dg, uint16_t *out)
{
    const uint32_t tid = threadIdx.x;
    const uint32_t ngrp = NT / dg, d = tid % dg, grp = tid / dg;
    float s = 0.f;
    if (grp < ngrp)
        for (uint32_t r = grp; r < rpp; r += ngrp)
            s += part[r * dg + d];
    __syncthreads();
    if (grp < ngrp)
        part[grp * dg + d] = s;
    __syncthreads();
    if (tid < dg)
    {
        float o = 0.f;
        for (uint32_t k = 0; k < ngrp && k < rpp; ++k)
            o += part[k * dg + tid];
        out[tid] = f2h(o);
    }
}

// block b -> (head, dim group): the G blocks of a head get consecutive ids with equal b % 8, i.e. one XCD and its
// L2, so the keys they all score and the partial lines of V rows they read are fetched from HBM once
__device__ __forceinline__ void block_head(uint32_t b, uint32_t G, uint32_t &h, uint32_t &g)
{
    h = (b % 8) + 8 * (b / (8 * G));
    g = (b / 8) % G;
}

// ---------------------------------------------------------------------------------------------------------------
// long caches, kernel 1: block (h, c) scores positions [c chunk, (c + 1) chunk) of head h
__global__ __launch_bounds__(256) void attn_scores_kernel(AttnDecodeArgs a)
{
    extern __shared__ float sm[]; // this chunk's scores
    __shared__ float rmax[4], rsum[4];
    const uint32_t h = blockIdx.x / a.cmax, c = blockIdx.x % a.cmax;
    const uint32_t kv = a.step->offset + 1;
    const uint32_t j0 = c * a.chunk;
    if (j0 >= kv)
        return;
    const uint32_t tid = threadIdx.x;
    const uint32_t n = min(a.chunk, kv - j0);
    const KeyLayout k = key_layout<256>(a.q + (size_t)h * a.hd, a.hd);
    const u32x4 *Kv = (const u32x4 *)(a.kc + ((size_t)h * a.ctx + j0) * a.hd);
    constexpr int U = 8; // 256 keys per round trip at head_dim 128
    for (uint32_t jb = k.ks; jb < n; jb += k.kpp * U)
    {
        u32x4 ka[U], kb[U];
        load_keys<U>(k, Kv, jb, n - 1, ka, kb);
        score_keys<U>(k, ka, kb, jb, n, a.scale, sm);
    }
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

// long caches, kernel 2: block (h, c) forms the chunk's partial sum o_c[d] = sum_{j in chunk} p_j v_j[d] with the
// row's probabilities p_j = fp16(exp(s_j - M) / L) (M, L reduced from all chunk statistics, identically in every
// block of the head); whole 16-byte vectors of contiguous rows, 16 lanes per 128-dim row
__global__ __launch_bounds__(256) void attn_pvc_kernel(AttnDecodeArgs a)
{
    __shared__ float rmax[4], rsum[4];
    __shared__ float pl[1024];
    __shared__ float part[2048];
    const uint32_t h = blockIdx.x / a.cmax, c = blockIdx.x % a.cmax;
    const uint32_t kv = a.step->offset + 1;
    const uint32_t j0 = c * a.chunk;
    if (j0 >= kv)
        return;
    const uint32_t tid = threadIdx.x;
    const uint32_t n = min(a.chunk, kv - j0), nc = (kv + a.chunk - 1) / a.chunk;
    const float *st = a.stats + (size_t)h * a.cmax * 2;
    const float *S = a.scores + (size_t)h * a.ctx;
    const uint16_t *Vh = a.vc + (size_t)h * a.ctx * a.hd;
    const uint32_t vpr = a.hd / 8, lpr = lanes_pow2(vpr), rpp = 256 / lpr;
    const uint32_t kl = tid % lpr, ks = tid / lpr;
    // statistics first, then this chunk's V rows and scores (counters retire in issue order)
    const uint32_t ci = min(tid, nc - 1);
    const float mc_raw = st[2 * ci], lc_raw = st[2 * ci + 1];
    constexpr int U = 16; // 256 rows per round trip at head_dim 128
    const u32x4 *Vv = (const u32x4 *)(Vh + (size_t)j0 * a.hd) + min(kl, vpr - 1);
    u32x4 vv[U];
#pragma unroll
    for (int t = 0; t < U; ++t)
        vv[t] = Vv[(size_t)min(ks + rpp * t, n - 1) * vpr];
    float sc = 0.f;
    if (tid < n)
        sc = S[j0 + tid];
    const float mc = tid < nc ? mc_raw : -FLT_MAX;
    const float M = block4_max(mc, rmax);
    const float L = block4_sum(tid < nc ? lc_raw * expf(mc - M) : 0.f, rsum);
    if (kv == a.hd)
    {
        // the transposed product needs every position: block 0 forms the whole output (one chunk when
        // chunk >= hd, else this reads the other chunks' scores, which the scores kernel has written)
        if (c != 0)
            return;
        for (uint32_t j = tid; j < kv; j += 256)
            pl[j] = h2f(f2h(expf(S[j] - M) / L));
        __syncthreads();
        pv_transposed(pl, Vh, a.out + (size_t)h * a.hd, kv, a.hd, 0, a.hd);
        return;
    }
    for (uint32_t j = tid; j < n; j += 256)
        pl[j] = h2f(f2h(expf((j == tid ? sc : S[j0 + j]) - M) / L));
    __syncthreads();
    float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    for (uint32_t jb = ks; jb < n; jb += rpp * U)
    {
        if (jb != ks)
        {
#pragma unroll
            for (int t = 0; t < U; ++t)
                vv[t] = Vv[(size_t)min(jb + rpp * t, n - 1) * vpr];
        }
#pragma unroll
        for (int t = 0; t < U; ++t)
        {
            const uint32_t j = jb + rpp * t;
            const float pj = j < n ? pl[j] : 0.f;
#pragma unroll
            for (int e = 0; e < 4; ++e)
            {
                acc[2 * e] = fmaf(pj, half_lo(vv[t][e]), acc[2 * e]);
                acc[2 * e + 1] = fmaf(pj, half_hi(vv[t][e]), acc[2 * e + 1]);
            }
        }
    }
    if (kl < vpr)
#pragma unroll
        for (int e = 0; e < 8; ++e)
            part[ks * a.hd + kl * 8 + e] = acc[e]; // rpp * hd <= 256 * 8
    __syncthreads();
    float o = 0.f;
    if (tid < a.hd)
        for (uint32_t k = 0; k < rpp; ++k)
            o += part[k * a.hd + tid];
    uint16_t *out = a.out + (size_t)h * a.hd;
    if (nc == 1)
    {
        if (tid < a.hd)
            out[tid] = f2h(o);
        return;
    }
    // Merge without a device-wide fence: the partials go out as agent-scope atomic stores (written through to the
    // level all XCDs share), every thread waits for its stores to complete, then one arrival is counted. The block
    // that arrives last reads the partials back with agent-scope atomic loads, adds them in chunk order and resets
    // the counter for the next launch. No block ever waits on another.
    float *P = a.part + (size_t)h * a.cmax * a.hd;
    if (tid < a.hd)
        __hip_atomic_store(P + (size_t)c * a.hd + tid, o, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    __shared__ uint32_t arrivals;
    if (tid == 0)
        arrivals = __hip_atomic_fetch_add(a.count + h, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __syncthreads();
    if (arrivals != nc - 1)
        return;
    // thread (s, d) adds partials i == s (mod ns), eight independent loads at a time; then the ns sums in order
    const uint32_t ns = 256 / a.hd > 0 ? 256 / a.hd : 1, sg = tid / a.hd, d = tid % a.hd;
    if (sg < ns)
    {
        float sum = 0.f;
        for (uint32_t i0 = sg; i0 < nc; i0 += 8 * ns)
        {
            float v[8];
#pragma unroll
            for (int u = 0; u < 8; ++u)
                v[u] = __hip_atomic_load(P + (size_t)min(i0 + ns * u, nc - 1) * a.hd + d, __ATOMIC_RELAXED,
                                         __HIP_MEMORY_SCOPE_AGENT);
#pragma unroll
            for (int u = 0; u < 8; ++u)
                sum += i0 + ns * u < nc ? v[u] : 0.f;
        }
        part[sg * a.hd + d] = sum;
    }
    __syncthreads();
    if (tid < a.hd)
    {
        float sum = 0.f;
        for (uint32_t k = 0; k < ns; ++k)
            sum += part[k * a.hd + tid];
        out[tid] = f2h(sum);
    }
    if (tid == 0)
        __hip_atomic_store(a.count + h, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// ---------------------------------------------------------------------------------------------------------------
// short caches: one kernel of 1024 threads per block (16 waves: the work is latency-bound, so each thread's share is
// short and four waves per SIMD interleave); LDS holds kv floats of scores, then probabilities
constexpr int kSmallThreads = 1024;

__device__ __forceinline__ float block16_max(float v, float *red)
{
    v = wave_max_dpp(v);
    if ((threadIdx.x & 63) == 0)
        red[threadIdx.x >> 6] = v;
    __syncthreads();
    float r = red[0];
#pragma unroll
    for (int i = 1; i < 16; ++i)
        r = fmaxf(r, red[i]);
    return r;
}
__device__ __forceinline__ float block16_sum(float v, float *red)
{
    v = wave_sum_dpp(v);
    if ((threadIdx.x & 63) == 0)
        red[threadIdx.x >> 6] = v;
    __syncthreads();
    float r = 0.f;
#pragma unroll
    for (int i = 0; i < 16; ++i)
        r += red[i];
    return r;
}

__global__ __launch_bounds__(kSmallThreads) void attn_decode_small_kernel(AttnDecodeArgs a)
{
    constexpr int NT = kSmallThreads;
    extern __shared__ float sm[];
    __shared__ float rmax[16], rsum[16];
    __shared__ float part[NT * 8];
    uint32_t h, g;
    block_head(blockIdx.x, a.groups, h, g);
    if (h >= a.H)
        return;
    const uint32_t tid = threadIdx.x;
    const uint32_t kv = a.step->offset + 1;
    const uint16_t *Vh = a.vc + (size_t)h * a.ctx * a.hd;
    const uint32_t dg = a.hd / a.groups, d0 = g * dg;
    const uint32_t lpr = dg / 8, vpr = a.hd / 8, rpp = NT / lpr;
    const uint32_t vl = tid % lpr, vs = tid / lpr;
    const u32x4 *Vv = (const u32x4 *)Vh + d0 / 8 + vl;
    // the block's first V rows are in flight while the keys are scored
    constexpr int UV = 1, U = 4;
    u32x4 vv[UV];
#pragma unroll
    for (int t = 0; t < UV; ++t)
        vv[t] = Vv[(size_t)min(vs + rpp * t, kv - 1) * vpr];
    const KeyLayout k = key_layout<NT>(a.q + (size_t)h * a.hd, a.hd);
    const u32x4 *Kv = (const u32x4 *)(a.kc + (size_t)h * a.ctx * a.hd);
    for (uint32_t jb = k.ks; jb < kv; jb += k.kpp * U)
    {
        u32x4 ka[U], kb[U];
        load_keys<U>(k, Kv, jb, kv - 1, ka, kb);
        score_keys<U>(k, ka, kb, jb, kv, a.scale, sm);
    }
    __syncthreads();
    float mx = -FLT_MAX;
    for (uint32_t j = tid; j < kv; j += NT)
        mx = fmaxf(mx, sm[j]);
    const float M = block16_max(mx, rmax);
    float sum = 0.f;
    for (uint32_t j = tid; j < kv; j += NT)
        sum += expf(sm[j] - M);
    const float L = block16_sum(sum, rsum);
    for (uint32_t j = tid; j < kv; j += NT)
        sm[j] = h2f(f2h(expf(sm[j] - M) / L));
    __syncthreads();
    uint16_t *out = a.out + (size_t)h * a.hd + d0;
    if (kv == a.hd)
    {
        pv_transposed(sm, Vh, out, kv, a.hd, d0, dg);
        return;
    }
    float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    for (uint32_t jb = vs; jb < kv; jb += rpp * UV)
    {
        if (jb != vs)
        {
#pragma unroll
            for (int t = 0; t < UV; ++t)
                vv[t] = Vv[(size_t)min(jb + rpp * t, kv - 1) * vpr];
        }
#pragma unroll
        for (int t = 0; t < UV; ++t)
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
    if (vs < rpp)
#pragma unroll
        for (int e = 0; e < 8; ++e)
            part[vs * dg + vl * 8 + e] = acc[e]; // rpp * dg <= NT * 8
    __syncthreads();
    pv_reduce_out<NT>(part, rpp, dg, out);
}

// ---------------------------------------------------------------------------------------------------------------
uint32_t attn_groups(uint32_t H, uint32_t hd, uint32_t max_groups)
{
    // the largest divisor of the row's 16-byte vectors that is <= max_groups while H * G stays <= 1024 blocks
    uint32_t best = 1;
    for (uint32_t g = 1; g <= max_groups; ++g)
        if ((hd / 8) % g == 0 && H * g <= 1024)
            best = g;
    return best;
}

static bool attn_args_ok(const AttnDecodeArgs &a)
{
    return a.hd % 8 == 0 && a.hd <= 256 && a.H > 0 && a.ctx > 0 && a.groups > 0 && (a.hd / 8) % a.groups == 0;
}

hipError_t launch_attn_scores(hipStream_t st, const AttnDecodeArgs &a)
{
    if (!attn_args_ok(a) || a.cmax == 0 || a.chunk == 0 || (uint64_t)a.chunk * a.cmax < a.ctx)
        return hipErrorInvalidValue;
    attn_scores_kernel<<<a.H * a.cmax, 256, (size_t)a.chunk * sizeof(float), st>>>(a);
    return hipGetLastError();
}

hipError_t launch_attn_pv(hipStream_t st, const AttnDecodeArgs &a)
{
    // pl holds a chunk's probabilities (or, for the transposed product, hd of them)
    if (!attn_args_ok(a) || a.cmax == 0 || a.chunk == 0 || a.chunk > 1024 || (uint64_t)a.chunk * a.cmax < a.ctx ||
        a.cmax > 256 || !a.part || !a.count)
        return hipErrorInvalidValue;
    attn_pvc_kernel<<<a.H * a.cmax, 256, 0, st>>>(a);
    return hipGetLastError();
}

hipError_t launch_attn_small(hipStream_t st, const AttnDecodeArgs &a, uint32_t kv_max)
{
    if (!attn_args_ok(a) || kv_max == 0 || kv_max > a.ctx)
        return hipErrorInvalidValue;
    attn_decode_small_kernel<<<(a.H + 7) / 8 * 8 * a.groups, kSmallThreads, (size_t)kv_max * sizeof(float), st>>>(a);
    return hipGetLastError();
}

} // namespace vk
