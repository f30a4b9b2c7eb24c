// Device pieces shared by the decode GEMV kernels (one launch per product, and the persistent decode step).
#pragma once

#include "device_common.h"
#include "kernels.h"

namespace vk
{

// EPI_ARGMAX after the workgroup's last unit: (bv, bi) is lane 0's best of its wave's rows. The workgroup's best goes
// out as agent-scope stores (written through to the level every XCD reads) and, once they are complete, one arrival
// is counted: workgroup b on counter b % G (G = min(grid, kArgmaxCounters)), and the last arrival on each of those
// counts once on the top counter. The workgroup that arrives last there reads every candidate back with agent-scope
// loads, eight per thread in flight, reduces them (the order is total, so the grouping does not matter) and clears
// the counters for the next launch. Arrivals on one word are serialised by its memory channel (about 10 ns each), so
// a grid of 2000 workgroups on one counter spent ~20 us in them; spread over 16 words they overlap.
__device__ __forceinline__ void gemv_argmax_finish(const GemvArgs &a, float bv, uint32_t bi)
{
    __shared__ float cv[4];
    __shared__ uint32_t ci[4];
    __shared__ uint32_t last;
    const uint32_t tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
    if (lane == 0)
    {
        cv[wid] = bv;
        ci[wid] = bi;
    }
    __syncthreads();
    if (tid == 0)
    {
        float v = cv[0];
        uint32_t i = ci[0];
        for (int w = 1; w < 4; ++w)
            if (am_before(cv[w], ci[w], v, i))
            {
                v = cv[w];
                i = ci[w];
            }
        // Release without a release fence: an agent-scope release compiles to buffer_wbl2 (a write-back of the
        // whole XCD L2) followed by a vmcnt(0) wait. The write-back is only needed for stores that were not written
        // through; these two are agent-scope atomic stores (sc1, written through to the level every XCD reads), so
        // the wait for their completion before the arrival is the whole of what the release has to provide.
        __hip_atomic_store(a.am_val + blockIdx.x, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(a.am_idx + blockIdx.x, i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __builtin_amdgcn_s_waitcnt(0);
        const uint32_t G = gridDim.x < kArgmaxCounters ? gridDim.x : kArgmaxCounters, c = blockIdx.x % G;
        const uint32_t in_c = gridDim.x / G + (c < gridDim.x % G ? 1u : 0u); // workgroups counted on counter c
        last = __hip_atomic_fetch_add(a.am_count + kArgmaxStride * c, 1u, __ATOMIC_RELAXED,
                                      __HIP_MEMORY_SCOPE_AGENT) == in_c - 1 &&
               __hip_atomic_fetch_add(a.am_count + kArgmaxStride * kArgmaxCounters, 1u, __ATOMIC_RELAXED,
                                      __HIP_MEMORY_SCOPE_AGENT) == G - 1;
    }
    __syncthreads();
    if (!last)
        return;
    // the last workgroup acquires what every other workgroup published (one cache invalidate, in one workgroup)
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
    float v = -INFINITY;
    uint32_t i = 0xFFFFFFFFu;
    constexpr uint32_t kBatch = 8;
    for (uint32_t j0 = tid; j0 < gridDim.x; j0 += 256 * kBatch)
    {
        // every load of a batch is issued before any compare waits for one (indices past the grid re-read the last
        // candidate and are skipped)
        float w[kBatch];
        uint32_t k[kBatch];
#pragma unroll
        for (uint32_t u = 0; u < kBatch; ++u)
        {
            const uint32_t j = min(j0 + 256 * u, gridDim.x - 1);
            w[u] = __hip_atomic_load(a.am_val + j, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            k[u] = __hip_atomic_load(a.am_idx + j, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
#pragma unroll
        for (uint32_t u = 0; u < kBatch; ++u)
            if (j0 + 256 * u < gridDim.x && am_before(w[u], k[u], v, i))
            {
                v = w[u];
                i = k[u];
            }
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1)
    {
        const float w = __shfl_xor(v, o, kWave);
        const uint32_t k = (uint32_t)__shfl_xor((int)i, o, kWave);
        if (am_before(w, k, v, i))
        {
            v = w;
            i = k;
        }
    }
    if (lane == 0)
    {
        cv[wid] = v;
        ci[wid] = i;
    }
    __syncthreads();
    if (tid == 0)
    {
        for (int w = 1; w < 4; ++w)
            if (am_before(cv[w], ci[w], v, i))
            {
                v = cv[w];
                i = ci[w];
            }
        a.am_ids[0] = i;
        if (a.am_io)
            a.am_io->id = i;
        for (uint32_t c = 0; c <= kArgmaxCounters; ++c)
            __hip_atomic_store(a.am_count + kArgmaxStride * c, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}

} // namespace vk
