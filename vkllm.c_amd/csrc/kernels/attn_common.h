// Device helpers shared by the decode attention kernels: how a workgroup's lanes split a cache row when scoring keys,
// how blocks map to (head, dim slice), and the short-cache kernel's launch constants.
#pragma once

#include "device_common.h"

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

} // namespace vk
