// Decode attention of the LLaMA-2 token step: one query row per head against the KV cache
// (src/models/vkllm_llama2_layers.c:223-257 with src/shaders/vkllm_softmax.comp:42-96 and
// src/shaders/vkllm_mat_mul_vec.comp:94-150 for the two products).
//
// The reference materialises fp16 scores, fp16 probabilities and an fp16 attention output, so each probability is
// rounded with the GLOBAL max and sum of its row. Both paths keep those rounding points:
//   short caches (one kernel, attn_decode_small_kernel): block (h, g) scores all kv keys of head h itself, reduces
//     the softmax statistics in the block and forms the probability-weighted sum for its slice of the head's dims.
//     attn_o_kernel runs the same blocks and the output projection in one launch.
//   long caches (fixed chunks of `chunk` positions): attn_scores_kernel writes fp16-rounded scores and each chunk's
//     max and sum of exp; attn_pvc_kernel reduces those statistics (identically in every block of the head),
//     rounds the chunk's probabilities, forms its partial sums, and the last chunk block of a head to finish adds
//     the partials in chunk order. attn_long_kernel does both in one launch when every chunk block fits on the
//     device at once.
// No kernel uses a device-wide fence (on this GPU one writes back a whole L2); kv == hd takes the reference's
// transposed product p . V^T.
#include <float.h>

#include <algorithm>

#include "attn_common.h"
#include "device_common.h"
#include "kernels.h"

namespace vk
{

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
// long caches, one kernel: block (h, c) does attn_scores_kernel's and attn_pvc_kernel's work for chunk c with the
// same arithmetic in the same order, so the output is identical. Its K and V rows (one round trip each at head_dim
// <= 128) are requested together at the start; the scores stay in LDS; the chunk's statistics go out as
// agent-scope stores and are counted on the head's counter, and the block waits (bounded) until every live chunk
// of the head has counted before it reduces them. The partial sums are then merged as in attn_pvc_kernel, on the
// same counter (a second round of arrivals); the merging block clears it. The launcher admits the launch only when
// every block can be resident at once.

__global__ __launch_bounds__(256) void attn_long_kernel(AttnDecodeArgs a)
{
    extern __shared__ float sm[]; // this chunk's scores
    __shared__ float rmax[4], rsum[4];
    __shared__ float pl[1024];
    __shared__ float part[2048];
    __shared__ uint32_t arrivals, gave_up;
    const uint32_t h = blockIdx.x / a.cmax, c = blockIdx.x % a.cmax;
    const uint32_t kv = a.step->offset + 1;
    const uint32_t j0 = c * a.chunk;
    if (j0 >= kv)
        return;
    const uint32_t tid = threadIdx.x;
    const uint32_t n = min(a.chunk, kv - j0), nc = (kv + a.chunk - 1) / a.chunk;
    uint32_t *const ctr = a.long_sync + (size_t)h * kAttnLongStride;
    float *const st = a.stats + (size_t)h * a.cmax * 2;
    const uint16_t *Vh = a.vc + (size_t)h * a.ctx * a.hd;

    // K rows of the chunk, then its scores; the V rows are requested only once the keys are in, so the keys of all
    // chunks (which gate the statistics exchange) do not share the memory system with V, and V streams in while the
    // statistics are exchanged
    const KeyLayout k = key_layout<256>(a.q + (size_t)h * a.hd, a.hd);
    const u32x4 *Kv = (const u32x4 *)(a.kc + ((size_t)h * a.ctx + j0) * a.hd);
    constexpr int U = 8, UV = 16; // keys and V rows per thread: 256 of each per round trip at head_dim 128
    u32x4 ka[U], kb[U];
    load_keys<U>(k, Kv, k.ks, n - 1, ka, kb);

    // scores and the chunk's statistics (attn_scores_kernel)
    score_keys<U>(k, ka, kb, k.ks, n, a.scale, sm);
    const uint32_t vpr = a.hd / 8, lpr = lanes_pow2(vpr), rpp = 256 / lpr;
    const uint32_t kl = tid % lpr, ks = tid / lpr;
    const u32x4 *Vv = (const u32x4 *)(Vh + (size_t)j0 * a.hd) + min(kl, vpr - 1);
    u32x4 vv[UV];
#pragma unroll
    for (int t = 0; t < UV; ++t)
        vv[t] = Vv[(size_t)min(ks + rpp * t, n - 1) * vpr];
    __syncthreads();
    float mx = -FLT_MAX;
    for (uint32_t j = tid; j < n; j += 256)
        mx = fmaxf(mx, sm[j]);
    mx = block4_max(mx, rmax);
    float sum = 0.f;
    for (uint32_t j = tid; j < n; j += 256)
        sum += expf(sm[j] - mx);
    sum = block4_sum(sum, rsum);
    if (tid == 0)
    {
        __hip_atomic_store(st + 2 * c, mx, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(st + 2 * c + 1, sum, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __builtin_amdgcn_s_waitcnt(0);
        __hip_atomic_fetch_add(ctr, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        uint32_t spins = 0, failed = a.spin_limit == 0 ? 1u : 0u;
        while (!failed && __hip_atomic_load(ctr, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) < nc)
        {
            if (++spins >= a.spin_limit)
            {
                failed = 1;
                break;
            }
            __builtin_amdgcn_s_sleep(1);
        }
        gave_up = failed;
    }
    __syncthreads();
    if (gave_up)
    {
        if (tid == 0)
            __hip_atomic_store(a.err, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
        return;
    }

    // the row's statistics, probabilities and this chunk's partial sums (attn_pvc_kernel)
    const uint32_t ci = min(tid, nc - 1);
    const float mc_raw = __hip_atomic_load(st + 2 * ci, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const float lc_raw = __hip_atomic_load(st + 2 * ci + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const float mc = tid < nc ? mc_raw : -FLT_MAX;
    const float M = block4_max(mc, rmax);
    const float L = block4_sum(tid < nc ? lc_raw * expf(mc - M) : 0.f, rsum);
    uint16_t *out = a.out + (size_t)h * a.hd;
    if (nc == 1 && tid == 0)
        __hip_atomic_store(ctr, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); // no merge round follows
    if (kv == a.hd)
    {
        // the transposed product needs every position: one chunk (the launcher admits chunk >= head_dim)
        for (uint32_t j = tid; j < kv; j += 256)
            pl[j] = h2f(f2h(expf(sm[j] - M) / L));
        __syncthreads();
        pv_transposed(pl, Vh, out, kv, a.hd, 0, a.hd);
        return;
    }
    for (uint32_t j = tid; j < n; j += 256)
        pl[j] = h2f(f2h(expf(sm[j] - M) / L));
    __syncthreads();
    float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int t = 0; t < UV; ++t)
    {
        const uint32_t j = ks + rpp * t;
        const float pj = j < n ? pl[j] : 0.f;
#pragma unroll
        for (int e = 0; e < 4; ++e)
        {
            acc[2 * e] = fmaf(pj, half_lo(vv[t][e]), acc[2 * e]);
            acc[2 * e + 1] = fmaf(pj, half_hi(vv[t][e]), acc[2 * e + 1]);
        }
    }
    if (kl < vpr)
#pragma unroll
        for (int e = 0; e < 8; ++e)
            part[ks * a.hd + kl * 8 + e] = acc[e];
    __syncthreads();
    float o = 0.f;
    if (tid < a.hd)
        for (uint32_t r = 0; r < rpp; ++r)
            o += part[r * a.hd + tid];
    if (nc == 1)
    {
        if (tid < a.hd)
            out[tid] = f2h(o);
        return;
    }
    // merge: the second round of arrivals on the head's counter; the last block adds the partials in chunk order
    float *P = a.part + (size_t)h * a.cmax * a.hd;
    if (tid < a.hd)
        __hip_atomic_store(P + (size_t)c * a.hd + tid, o, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (tid == 0)
        arrivals = __hip_atomic_fetch_add(ctr, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __syncthreads();
    if (arrivals != 2 * nc - 1)
        return;
    const uint32_t ns = 256 / a.hd > 0 ? 256 / a.hd : 1, sg = tid / a.hd, d = tid % a.hd;
    if (sg < ns)
    {
        float total = 0.f;
        for (uint32_t i0 = sg; i0 < nc; i0 += 8 * ns)
        {
            float v[8];
#pragma unroll
            for (int u = 0; u < 8; ++u)
                v[u] = __hip_atomic_load(P + (size_t)min(i0 + ns * u, nc - 1) * a.hd + d, __ATOMIC_RELAXED,
                                         __HIP_MEMORY_SCOPE_AGENT);
#pragma unroll
            for (int u = 0; u < 8; ++u)
                total += i0 + ns * u < nc ? v[u] : 0.f;
        }
        part[sg * a.hd + d] = total;
    }
    __syncthreads();
    if (tid < a.hd)
    {
        float total = 0.f;
        for (uint32_t r = 0; r < ns; ++r)
            total += part[r * a.hd + tid];
        out[tid] = f2h(total);
    }
    if (tid == 0)
        __hip_atomic_store(ctr, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// ---------------------------------------------------------------------------------------------------------------
// block b of the short-cache attention (blocks of heads >= H do nothing; a position past the launch's small_max
// raises the step's error flag, in small_block)
template <bool AGENT, int UK = 4, int NB = 2, int VPRE = 2>
__device__ __forceinline__ void small_attention(const AttnDecodeArgs &a, uint32_t b, float *sm, float *red)
{
    uint32_t h, g;
    block_head(b, a.groups, h, g);
    if (h >= a.H)
        return;
    small_block<kSmallThreads, AGENT, NoHook, UK, NB, VPRE>(a, h, g, sm, red);
}

template <int UK, int NB, int VPRE>
__global__ __launch_bounds__(kSmallThreads) void attn_decode_small_kernel(AttnDecodeArgs a)
{
    extern __shared__ float sm[];
    __shared__ float red[kSmallRed];
    small_attention<false, UK, NB, VPRE>(a, blockIdx.x, sm, red);
}

// ---------------------------------------------------------------------------------------------------------------
// Short-cache attention and the output projection with its residual add (src/models/vkllm_llama2_layers.c:247-301)
// in one launch. The projection's 2 D^2 bytes of weights do not depend on the attention output, so they stream
// from HBM while the (latency-bound) attention runs:
//   blocks [0, A): the attention blocks above. Each writes its slice of the attention output with agent-scope
//     stores and waits for them to complete; then block b counts one arrival in counter b % 8, the last arrival of
//     each counter counts one in `top`, and the last of those raises `ready`. (Arrivals spread over 8 counters and
//     a flag that only the waiting side reads keep the atomics from queueing behind each other and the polls.)
//   blocks [A, grid): Wo rows, two per wave unit. After about a microsecond (the attention's own cache reads go
//     first) the first unit's weights are requested; thread 0 then waits (bounded) for `ready`, the block reads the
//     attention output with agent-scope loads, and the rows are finished as the separate GEMV does:
//     out[r] = fp16(resid[r] + fp16(Wo[r] . attn)). The last of these blocks to finish clears the counters.
// Attention blocks never wait, and the launcher sizes the grid so that every block is resident at once. A wait that
// gives up sets *err (the step's outputs are then not valid).
// sync words: arrival counters at kSyncStride c (c < 8), then top, ready and done, each on its own 256 bytes
constexpr uint32_t kSyncStride = 64;
constexpr uint32_t kSyncTop = 8 * kSyncStride, kSyncReady = 9 * kSyncStride, kSyncDone = 10 * kSyncStride;
static_assert(kSyncDone < kAttnSyncWords, "sync words");

template <int NV> __global__ __launch_bounds__(kSmallThreads, 4) void attn_o_kernel(AttnOArgs a)
{
    extern __shared__ float sm[]; // attention: kv scores; projection: the attention output (D halves)
    __shared__ float red[kSmallRed];
    __shared__ uint32_t gave_up;
    constexpr uint32_t NW = kSmallThreads / 64;
    const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    uint32_t *const top = a.sync + kSyncTop, *const ready = a.sync + kSyncReady, *const done = a.sync + kSyncDone;
    const uint32_t A = a.attn_blocks;
    if (blockIdx.x < A)
    {
        small_attention<true>(a.at, blockIdx.x, sm, red);
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
        if (tid == 0)
        {
            const uint32_t c = blockIdx.x % 8, groups = A < 8 ? A : 8;
            const uint32_t in_c = A / 8 + (c < A % 8 ? 1u : 0u); // attention blocks counted by counter c
            if (__hip_atomic_fetch_add(a.sync + kSyncStride * c, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
                    in_c - 1 &&
                __hip_atomic_fetch_add(top, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == groups - 1)
                __hip_atomic_store(ready, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        return;
    }
    const uint32_t D = a.at.H * a.at.hd, nvec = D / 8, units = D / 2;
    const uint32_t nblk = gridDim.x - A, stride = nblk * NW;
    uint32_t u = (blockIdx.x - A) * NW + wave;
    u32x4 w[2][NV];
    auto load_unit = [&](uint32_t unit) {
#pragma unroll
        for (int k = 0; k < 2; ++k)
        {
            // rows of units past the end read row 0; their sums are never stored
            const uint32_t row = unit < units ? 2 * unit + k : 0;
            const u32x4 *wr = (const u32x4 *)(a.wo + (size_t)row * D);
#pragma unroll
            for (int i = 0; i < NV; ++i)
                w[k][i] = __builtin_nontemporal_load(wr + min(lane + 64 * i, nvec - 1));
        }
    };
    {
        // about 1 us of the 100 MHz wall clock (bounded), so that the attention's reads are queued first
        const uint64_t t0 = wall_clock64();
        for (int i = 0; i < 64 && wall_clock64() - t0 < 100; ++i)
            __builtin_amdgcn_s_sleep(2);
    }
    load_unit(u);
    if (tid == 0)
    {
        uint32_t spins = 0, failed = a.at.spin_limit == 0 ? 1u : 0u;
        while (!failed && __hip_atomic_load(ready, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == 0u)
        {
            if (++spins >= a.at.spin_limit)
            {
                failed = 1;
                break;
            }
            __builtin_amdgcn_s_sleep(1);
        }
        gave_up = failed;
    }
    __syncthreads();
    uint32_t *xs = (uint32_t *)sm;
    const uint32_t *src = (const uint32_t *)a.at.out;
    for (uint32_t j = tid; j < D / 2; j += kSmallThreads)
        xs[j] = __hip_atomic_load(src + j, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __syncthreads();
    const u32x4 *xv = (const u32x4 *)sm;
    while (u < units)
    {
        float acc0 = 0.f, acc1 = 0.f;
#pragma unroll
        for (int i = 0; i < NV; ++i)
        {
            const uint32_t vi = lane + 64 * i;
            if (vi < nvec)
            {
                const u32x4 x = xv[vi];
                acc0 = dot8(w[0][i], x, acc0);
                acc1 = dot8(w[1][i], x, acc1);
            }
        }
        const uint32_t r = 2 * u;
        u += stride;
        if (u < units)
            load_unit(u);
        acc0 = wave_sum_dpp(acc0);
        acc1 = wave_sum_dpp(acc1);
        if (lane == 0)
        {
            a.out[r] = f2h(h2f(a.resid[r]) + h2f(f2h(acc0)));
            a.out[r + 1] = f2h(h2f(a.resid[r + 1]) + h2f(f2h(acc1)));
        }
    }
    // every block of the launch has passed its wait once all projection blocks are here: clear for the next launch
    __syncthreads();
    if (tid == 0)
    {
        if (gave_up)
            __hip_atomic_store(a.err, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
        if (__hip_atomic_fetch_add(done, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == nblk - 1)
        {
            for (uint32_t c = 0; c < 8; ++c)
                __hip_atomic_store(a.sync + kSyncStride * c, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(top, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(ready, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(done, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
}

// ---------------------------------------------------------------------------------------------------------------
uint32_t attn_groups(uint32_t H, uint32_t hd, uint32_t max_groups)
{
    // the largest divisor of the row's 16-byte vectors that is <= max_groups while H * G stays <= 1024 blocks
    uint32_t best = 1;
    for (uint32_t g = 1; g <= max_groups && g <= hd / 8; ++g)
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

bool attn_long_ok(const AttnDecodeArgs &a)
{
    // one round trip of keys and of V rows per block (head_dim <= 128 with chunks of <= 256 positions); the
    // transposed product (kv == hd) fits one chunk
    return attn_args_ok(a) && a.hd <= 128 && a.cmax > 0 && a.chunk >= a.hd && a.chunk <= 256 &&
           (uint64_t)a.chunk * a.cmax >= a.ctx && a.cmax <= 256;
}

hipError_t launch_attn_long(hipStream_t st, const AttnDecodeArgs &a, int cu_count)
{
    if (!attn_long_ok(a) || a.chunk == 0 || !a.part || !a.stats || !a.long_sync || !a.err)
        return hipErrorInvalidValue;
    const size_t lds = (size_t)a.chunk * sizeof(float);
    static uint64_t occ_memo = 0;
    const int per_cu = std::max(occupancy_per_cu((const void *)attn_long_kernel, 256, lds, occ_memo), 0);
    // the blocks of a head wait for each other: all of them must be resident at once
    if ((uint64_t)a.H * a.cmax > (uint64_t)(cu_count > 0 ? cu_count : 256) * (uint32_t)per_cu)
        return hipErrorInvalidConfiguration;
    attn_long_kernel<<<a.H * a.cmax, 256, lds, st>>>(a);
    return hipGetLastError();
}

uint32_t attn_small_limit(const AttnDecodeArgs &a)
{
    if (!attn_args_ok(a))
        return 0;
    // the slice's 16-byte vectors per row must split a wave evenly, and the P.V exchange holds 32 dims per wave
    const uint32_t lpr = a.hd / a.groups / 8;
    if (lpr != 1 && lpr != 2 && lpr != 4)
        return 0;
    return kSmallMaxPasses * (kSmallThreads / lpr);
}

static uint32_t small_blocks(const AttnDecodeArgs &a)
{
    return (a.H + 7) / 8 * 8 * a.groups;
}

hipError_t launch_attn_small(hipStream_t st, const AttnDecodeArgs &a, uint32_t kv_max)
{
    if (kv_max == 0 || kv_max > a.ctx || kv_max > attn_small_limit(a))
        return hipErrorInvalidValue;
    AttnDecodeArgs b = a;
    b.small_max = kv_max;
    // the keys and V rows requested before the position is known, sized to kv_max: per batch of keys a thread takes
    // UK rows kpp apart (one batch when kv_max <= 4 kpp, else two, the rest later); V passes of rpp rows (two at
    // most). Measured at the 7B widths and kv 150 (bucket bound 192): 128 KB of key rows per block requested, 38 KB
    // of them live, with the fixed two batches of four.
    uint32_t lpk = 1;
    while (lpk * 16 < a.hd)
        lpk <<= 1;
    const uint32_t kpp = kSmallThreads / lpk, dg = a.hd / a.groups, rpp = (kSmallThreads / 64) * (64 / (dg / 8));
    const uint32_t uk = (kv_max + kpp - 1) / kpp, vpre = (kv_max + rpp - 1) / rpp;
    const dim3 grid(small_blocks(a));
    const size_t lds = (size_t)kv_max * sizeof(float);
    if (uk > 4)
        attn_decode_small_kernel<4, 2, 2><<<grid, kSmallThreads, lds, st>>>(b);
    else if (vpre > 1)
        switch (uk)
        {
        case 1:
            attn_decode_small_kernel<1, 1, 2><<<grid, kSmallThreads, lds, st>>>(b);
            break;
        case 2:
            attn_decode_small_kernel<2, 1, 2><<<grid, kSmallThreads, lds, st>>>(b);
            break;
        case 3:
            attn_decode_small_kernel<3, 1, 2><<<grid, kSmallThreads, lds, st>>>(b);
            break;
        default:
            attn_decode_small_kernel<4, 1, 2><<<grid, kSmallThreads, lds, st>>>(b);
        }
    else
        switch (uk)
        {
        case 1:
            attn_decode_small_kernel<1, 1, 1><<<grid, kSmallThreads, lds, st>>>(b);
            break;
        case 2:
            attn_decode_small_kernel<2, 1, 1><<<grid, kSmallThreads, lds, st>>>(b);
            break;
        case 3:
            attn_decode_small_kernel<3, 1, 1><<<grid, kSmallThreads, lds, st>>>(b);
            break;
        default:
            attn_decode_small_kernel<4, 1, 1><<<grid, kSmallThreads, lds, st>>>(b);
        }
    return hipGetLastError();
}

// smallest compiled NV (16-byte vectors per lane and row) covering K = D
static int attn_o_nv(uint32_t D)
{
    static const int nv[] = {1, 2, 4, 8, 10};
    for (int v : nv)
        if ((uint32_t)v * 64 * 8 >= D)
            return v;
    return 0;
}

template <int NV> static hipError_t launch_attn_o_nv(hipStream_t st, AttnOArgs a, uint32_t kv_max, int cu_count)
{
    const uint32_t D = a.at.H * a.at.hd;
    const size_t lds = std::max((size_t)kv_max * sizeof(float), (size_t)D * 2);
    // resident blocks per CU at this LDS size (0 when the query fails, which rejects the launch)
    static uint64_t occ_memo = 0;
    const int per_cu = std::max(occupancy_per_cu((const void *)attn_o_kernel<NV>, kSmallThreads, lds, occ_memo), 0);
    const uint32_t cap = (uint32_t)(cu_count > 0 ? cu_count : 256) * (uint32_t)per_cu;
    const uint32_t A = small_blocks(a.at), units = D / 2, NW = kSmallThreads / 64;
    if (cap <= A)
        return hipErrorInvalidConfiguration;
    const uint32_t B = std::min(cap - A, (units + NW - 1) / NW);
    a.attn_blocks = A;
    a.at.small_max = kv_max;
    attn_o_kernel<NV><<<A + B, kSmallThreads, lds, st>>>(a);
    return hipGetLastError();
}

hipError_t launch_attn_o(hipStream_t st, const AttnOArgs &a, uint32_t kv_max, int cu_count)
{
    const uint32_t D = a.at.H * a.at.hd;
    if (kv_max == 0 || kv_max > a.at.ctx || kv_max > attn_small_limit(a.at) || !a.wo || !a.resid || !a.out ||
        !a.sync || !a.err)
        return hipErrorInvalidValue;
    switch (attn_o_nv(D))
    {
    case 1:
        return launch_attn_o_nv<1>(st, a, kv_max, cu_count);
    case 2:
        return launch_attn_o_nv<2>(st, a, kv_max, cu_count);
    case 4:
        return launch_attn_o_nv<4>(st, a, kv_max, cu_count);
    case 8:
        return launch_attn_o_nv<8>(st, a, kv_max, cu_count);
    case 10:
        return launch_attn_o_nv<10>(st, a, kv_max, cu_count);
    default:
        return hipErrorInvalidValue;
    }
}

} // namespace vk
