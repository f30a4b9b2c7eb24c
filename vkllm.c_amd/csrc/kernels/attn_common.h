// Device helpers shared by the decode attention kernels: how a workgroup's lanes split a cache row when scoring keys,
// how blocks map to (head, dim slice), the short-cache kernel's launch constants, and its block (which the
// persistent decode step runs as its attention part).
#pragma once

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

// the layout's indices for NT threads; the query vectors are left for the caller
template <int NT> __device__ __forceinline__ KeyLayout key_layout_idx(uint32_t hd)
{
    KeyLayout k;
    k.vpr = hd / 8;
    k.lpk = key_lanes(hd);
    k.kl = threadIdx.x % k.lpk;
    k.ks = threadIdx.x / k.lpk;
    k.kpp = NT / k.lpk;
    k.c0 = min(2 * k.kl, k.vpr - 1);
    k.c1 = min(2 * k.kl + 1, k.vpr - 1);
    return k;
}

// zero the query vectors of lanes past the row
__device__ __forceinline__ void key_layout_mask(KeyLayout &k)
{
    if (2 * k.kl >= k.vpr)
        k.q0 = (u32x4){0, 0, 0, 0};
    if (2 * k.kl + 1 >= k.vpr)
        k.q1 = (u32x4){0, 0, 0, 0};
}

template <int NT> __device__ __forceinline__ KeyLayout key_layout(const uint16_t *q, uint32_t hd)
{
    KeyLayout k = key_layout_idx<NT>(hd);
    const u32x4 *qv = (const u32x4 *)q;
    k.q0 = qv[k.c0];
    k.q1 = qv[k.c1];
    key_layout_mask(k);
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

// block b -> (head, dim group): the G blocks of a head get consecutive ids with equal b % 8, i.e. one XCD and its
// L2, so the keys they all score and the partial lines of V rows they read are fetched from HBM once
__device__ __forceinline__ void block_head(uint32_t b, uint32_t G, uint32_t &h, uint32_t &g)
{
    h = (b % 8) + 8 * (b / (8 * G));
    g = (b / 8) % G;
}

// short caches: one block of 512 threads per (head, dim slice)
constexpr int kSmallThreads = 512;
constexpr int kSmallMaxPasses = 6; // V rows per thread; kv <= kSmallMaxPasses * (rows per pass)
constexpr int kSmallRed = (kSmallThreads / 64) * 32;

// sum over aligned segments of `seg` lanes (16, 32 or 64); the last lane of each segment holds its sum
__device__ __forceinline__ float seg_sum(float v, uint32_t seg)
{
    v = group_sum(v, 16);
    if (seg >= 32)
        v = dpp_add<0x142, 0xA>(v);
    if (seg >= 64)
        v = dpp_add<0x143, 0xC>(v);
    return v;
}

// two fp16 outputs as one 32-bit word; agent-scope (written through to the level all XCDs share) when another
// workgroup of the same launch reads them
template <bool AGENT> __device__ __forceinline__ void store_pair(uint16_t *p, float a, float b)
{
    const uint32_t v = pack2(f2h(a), f2h(b));
    if (AGENT)
        __hip_atomic_store((uint32_t *)p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    else
        *(uint32_t *)p = v;
}

// ---------------------------------------------------------------------------------------------------------------
// short caches: one block of 512 threads per (head, dim slice). The work is latency-bound: the block has its first
// keys and V rows in flight before it knows the position, each wave reduces the softmax statistics on its own, and
// the P.V partials are reduced inside each wave before one exchange through LDS. LDS holds kv floats of scores.
// the reference's transposed product (kv == hd): out[r] = fp16(sum_k p_k V[r][k]) for this block's rows, two per
// thread
template <bool AGENT>
__device__ __forceinline__ void pv_transposed_pairs(const float *pl, const uint16_t *Vh, uint16_t *out, uint32_t kv,
                                                    uint32_t hd, uint32_t d0, uint32_t dg)
{
    for (uint32_t r = 2 * threadIdx.x; r < dg; r += 2 * blockDim.x)
    {
        const uint16_t *row0 = Vh + (size_t)(d0 + r) * hd, *row1 = row0 + hd;
        float a0 = 0.f, a1 = 0.f;
        for (uint32_t k = 0; k < kv; ++k)
        {
            a0 = fmaf(pl[k], h2f(row0[k]), a0);
            a1 = fmaf(pl[k], h2f(row1[k]), a1);
        }
        store_pair<AGENT>(out + r, a0, a1);
    }
}

// Block (h, g) of the short-cache attention: all kv keys of head h scored, the softmax statistics, then the
// probability-weighted sum of dims [g dg, (g + 1) dg) of V.
// The first two batches of keys and two passes of V rows (512 positions at head_dim 128) are requested before the
// position is known, at rows clamped to the launch's largest cache length small_max (further V passes follow the
// keys): a launch for short caches asks HBM for no row past small_max, the clamped requests repeat a row already in
// flight. Rows at or past kv never reach a score or a sum (their scores are not stored and their V values are
// replaced by zeros, whatever the cache holds there). After the scores are in LDS every wave reduces the statistics
// itself, so no further exchange is needed until the P.V partials.
struct NoHook
{
    __device__ void operator()() const {}
};
// exp(x) as 2^(x log2 e) on the hardware exponential (v_exp_f32), as the prompt-step attention takes it (the
// reference's shader leaves exp to the implementation's precision); a block's softmax then costs a few cycles per
// score instead of the library expf's range reduction and polynomial
__device__ __forceinline__ float small_exp(float x)
{
    return __builtin_amdgcn_exp2f(x * 1.4426950408889634f);
}

// after_issue runs once the block's first keys and V rows are requested (the persistent step requests the next
// product's weights there, behind the cache reads).
// UK: key rows per thread in a batch (kpp UK keys per batch); NB: batches of keys requested before the position is
// read (2: the second is requested during the first's scores otherwise); VPRE: passes of V rows requested then.
// The launcher sizes them to the launch's bound small_max, so that a short cache asks for no more rows than it can
// hold (a row past small_max would only repeat the clamped last one).
template <int NT, bool AGENT, typename Hook = NoHook, int UK = 4, int NB = 2, int VPRE = 2>
__device__ __forceinline__ void small_block(const AttnDecodeArgs &a, uint32_t h, uint32_t g, float *sm, float *red,
                                            Hook after_issue = Hook())
{
    static_assert(UK >= 1 && UK <= 4 && (NB == 1 || NB == 2) && (VPRE == 1 || VPRE == 2), "speculative sizes");
    constexpr uint32_t NW = NT / 64;
    constexpr int U = UK, UV = kSmallMaxPasses;
    const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint32_t dg = a.hd / a.groups, d0 = g * dg, vpr = a.hd / 8, last = min(a.small_max, a.ctx) - 1;
    // V layout: lane = (vector vl of the slice, row slot); a wave covers seg rows, the block rpp rows per pass
    const uint32_t lpr = dg / 8, seg = 64 / lpr;
    const uint32_t vl = lane / seg, vs = wave * seg + lane % seg, rpp = NW * seg;
    const uint16_t *Vh = a.vc + (size_t)h * a.ctx * a.hd;
    const u32x4 *Vv = (const u32x4 *)Vh + d0 / 8 + vl;
    u32x4 vv[UV];
    vv[0] = Vv[(size_t)min(vs, last) * vpr];
    if constexpr (VPRE > 1)
        vv[1] = Vv[(size_t)min(vs + rpp, last) * vpr];
    const KeyLayout k = key_layout<NT>(a.q + (size_t)h * a.hd, a.hd);
    const u32x4 *Kv = (const u32x4 *)(a.kc + (size_t)h * a.ctx * a.hd);
    const uint32_t step = k.kpp * U;
    u32x4 ka[U], kb[U], na[U], nb[U];
    load_keys<U>(k, Kv, k.ks, last, ka, kb);
    if constexpr (NB > 1)
        load_keys<U>(k, Kv, k.ks + step, last, na, nb);
    after_issue();
    // the position is read only now, behind the cache rows (the reads above are clamped to small_max): a position
    // past small_max (the LDS's positions and the speculative loads' bound) is a host error, and the block raises
    // the step's error flag and writes nothing
    const uint32_t kv = a.step->offset + 1;
    if (kv > a.small_max)
    {
        if (tid == 0 && a.err)
            __hip_atomic_store(a.err, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
        return;
    }
    const uint32_t passes = (kv + rpp - 1) / rpp;
    const uint32_t nit = (kv + step - 1) / step;
    for (uint32_t it = 0; it < nit; ++it)
    {
        const bool more = it + 1 < nit; // block-uniform
        if constexpr (NB == 1)
            if (more)
                load_keys<U>(k, Kv, k.ks + (it + 1) * step, kv - 1, na, nb);
        score_keys<U>(k, ka, kb, k.ks + it * step, kv, a.scale, sm);
        if (more)
#pragma unroll
            for (int u = 0; u < U; ++u)
            {
                ka[u] = na[u];
                kb[u] = nb[u];
            }
        if constexpr (NB > 1)
            if (it + 2 < nit)
                load_keys<U>(k, Kv, k.ks + (it + 2) * step, kv - 1, na, nb);
    }
    // V rows past the passes requested at the start, once the key registers are free
#pragma unroll
    for (int t = VPRE; t < UV; ++t)
        if ((uint32_t)t < passes)
            vv[t] = Vv[(size_t)min(vs + rpp * t, kv - 1) * vpr];
    __syncthreads();
    // softmax statistics, reduced by every wave over all kv scores (same values, same order in each wave)
    float M = -FLT_MAX;
    for (uint32_t j = lane; j < kv; j += 64)
        M = fmaxf(M, sm[j]);
    M = wave_max_dpp(M);
    float L = 0.f;
    for (uint32_t j = lane; j < kv; j += 64)
        L += small_exp(sm[j] - M);
    L = wave_sum_dpp(L);
    uint16_t *out = a.out + (size_t)h * a.hd + d0;
    if (kv == a.hd)
    {
        __syncthreads(); // every wave has its statistics before the scores become probabilities
        for (uint32_t j = tid; j < kv; j += NT)
            sm[j] = h2f(f2h(small_exp(sm[j] - M) / L));
        __syncthreads();
        pv_transposed_pairs<AGENT>(sm, Vh, out, kv, a.hd, d0, dg);
        return;
    }
    float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int t = 0; t < UV; ++t)
    {
        const uint32_t j = vs + rpp * t;
        if ((uint32_t)t < passes) // block-uniform
        {
            const bool live = j < kv;
            const float pj = live ? h2f(f2h(small_exp(sm[min(j, kv - 1)] - M) / L)) : 0.f;
#pragma unroll
            for (int e = 0; e < 4; ++e)
            {
                const uint32_t v = live ? vv[t][e] : 0u;
                acc[2 * e] = fmaf(pj, half_lo(v), acc[2 * e]);
                acc[2 * e + 1] = fmaf(pj, half_hi(v), acc[2 * e + 1]);
            }
        }
    }
    float *part = red; // NW rows of dg partial sums
#pragma unroll
    for (int e = 0; e < 8; ++e)
        acc[e] = seg_sum(acc[e], seg);
    if (lane % seg == seg - 1)
#pragma unroll
        for (int e = 0; e < 8; ++e)
            part[wave * dg + vl * 8 + e] = acc[e];
    __syncthreads();
    if (2 * tid < dg)
    {
        float o0 = 0.f, o1 = 0.f;
#pragma unroll
        for (uint32_t w = 0; w < NW; ++w)
        {
            o0 += part[w * dg + 2 * tid];
            o1 += part[w * dg + 2 * tid + 1];
        }
        store_pair<AGENT>(out + 2 * tid, o0, o1);
    }
}

} // namespace vk
