// Persistent single-token step: the whole LLaMA-2 token step after the embedding (src/models/vkllm_llama2_layers.c:
// 98-354 per layer, src/models/vkllm_models_llama2.c:560-602 for the output norm, vocabulary product and arg max) in
// one launch of one or two workgroups per CU, all resident at once.
//
// Per layer the grid runs five phases, separated by grid barriers:
//   A  RMSNorm(h) -> [Wq;Wk;Wv] -> RoPE(q, k); q to qs[l], k and v into the caches at the step's position
//   B  single-token attention over the cache (the short-cache kernel's block, 256 threads per (head, dim slice))
//   C  h' = h + Wo attn
//   D  RMSNorm(h') -> [Wu;Wg] -> up * silu(gate)
//   E  h'' = h' + Wd act
// then the output RMSNorm, the vocabulary product and its arg max. Each phase computes exactly what the separate
// decode kernels compute, with the same per-lane vector assignment and summation order (the GEMV phases give the
// same bits; the attention's P.V partial sums are grouped by its 256-thread blocks).
//
// Why one launch: a decode step is a chain of small HBM-bound products, and between two launches the weight stream
// stops (the last waves drain, the next kernel starts and ramps up). Here a wave requests its first unit of the next
// phase's weights as soon as its own stores are done, before it waits at the barrier, so the weight stream runs on
// through the barrier; the next phase's input (a few KB) is what the wave waits for.
//
// Measured at the 7B shape it is slower than the separate launches (3.05 against 2.50 ms per token), so it runs only
// with VKLLM_PERSIST=1. Per-phase wall-clock stamps of one layer (92 us against 77 us for the five launches) showed
// where: every product streams at 6.2-6.4 TB/s inside its phase, but each barrier waits 1.2-2 us for the slowest
// workgroup (9.8 us after the gate/up phase, whose 11008 units do not divide over the 1024 waves), and the
// attention part takes 9 us (256-thread blocks, one wave per SIMD) against the 6 us of its own launch. The kernel
// needs more than 256 registers per wave (the phases' weights in flight, input rows and the attention all live in
// one function), so a CU holds one workgroup and each wave one unit in flight; two units per wave, or two
// workgroups per CU, spill to scratch and measured slower still (3.46 and 2.93 ms).
//
// Memory ordering without device-wide fences (on this GPU a release fence writes back a whole XCD L2):
//   - every value a later phase reads is stored with agent-scope stores (written through to the level all XCDs
//     share), and a workgroup arrives at a barrier only after s_waitcnt(0) in all of its waves;
//   - every activation row is written once per step into its own buffer (hs, qs, attns, acts) and read only after
//     the barrier that follows its phase, so no L2 can hold an older copy of a line a phase reads; the KV cache rows
//     of the step's position are likewise read only in their layer's attention phase;
//   - the barrier: arrivals spread over 8 counters (workgroup b counts in counter b % 8, one XCD each), the last
//     arrival of each counter counts in `top`, the last of those raises the flag to k + 1; waiters poll the flag.
//     Counts grow monotonically through the launch (every workgroup waits for barrier k before it arrives at k + 1),
//     and the last workgroup to finish clears every word.
// Every wait is bounded: a wait that gives up raises *err and an abort word, after which every wait returns at once,
// so every wave reaches the end of the kernel; the host then runs the step on the separate kernels.
#include <float.h>

#include <algorithm>

#include "attn_common.h"
#include "device_common.h"
#include "gemv_common.h"
#include "kernels.h"

namespace vk
{

namespace
{

constexpr uint32_t kPStride = 64; // sync words 256 bytes apart
constexpr uint32_t kPTop = 8 * kPStride, kPFlag = 9 * kPStride, kPDone = 10 * kPStride, kPAbort = 11 * kPStride;
static_assert(kPAbort < kPersistSyncWords, "sync words");

// the workgroup's arrival at barrier k (thread 0; every wave of the workgroup has waited for its stores)
__device__ __forceinline__ void arrive(const PersistArgs &a, uint32_t k)
{
    const uint32_t B = gridDim.x, c = blockIdx.x % 8, groups = B < 8 ? B : 8;
    const uint32_t in_c = B / 8 + (c < B % 8 ? 1u : 0u); // workgroups counted by counter c
    if (__hip_atomic_fetch_add(a.sync + kPStride * c, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) + 1 ==
            (k + 1) * in_c &&
        __hip_atomic_fetch_add(a.sync + kPTop, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) + 1 == (k + 1) * groups)
        __hip_atomic_store(a.sync + kPFlag, k + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// all threads: returns once barrier k is complete, or at once after any wait of the launch gave up
__device__ __forceinline__ void wait_barrier(const PersistArgs &a, uint32_t k)
{
    if (threadIdx.x == 0)
    {
        uint32_t spins = 0;
        while (__hip_atomic_load(a.sync + kPFlag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) < k + 1)
        {
            if ((spins & 63) == 0 && __hip_atomic_load(a.sync + kPAbort, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT))
                break;
            if (++spins >= a.spin_limit)
            {
                __hip_atomic_store(a.sync + kPAbort, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                __hip_atomic_store(a.err, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
                break;
            }
            __builtin_amdgcn_s_sleep(1);
        }
    }
    __syncthreads();
}

// end of a phase: this workgroup's stores are complete, then it arrives at barrier k (wave 0, before it requests
// anything: a returning atomic waits for every earlier request of its wave)
__device__ __forceinline__ void finish_phase(const PersistArgs &a, uint32_t k)
{
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (threadIdx.x == 0)
        arrive(a, k);
}

// NV 16-byte vectors per lane of weight row `row` (lane l: vectors l + 64 i, clamped into the row) into w[B + i]
template <int NV, int B, int WN>
__device__ __forceinline__ void load_row(u32x4 (&w)[WN], const uint16_t *W, size_t row, uint32_t nvec)
{
    // (lane through an empty asm: the per-lane offsets are recomputed at each request instead of being hoisted out
    // of the layer loop and held in registers through every phase)
    uint32_t lane = threadIdx.x & 63;
    asm volatile("" : "+v"(lane));
    const u32x4 *wr = (const u32x4 *)W + row * nvec;
#pragma unroll
    for (int i = 0; i < NV; ++i)
        w[B + i] = __builtin_nontemporal_load(wr + min(lane + 64 * i, nvec - 1));
}

// the input row x (K halves) into LDS as 16-byte vectors, RMS-normalised with weights nw when NORM (the GEMV
// kernel's prologue: thread t holds vectors t + 256 i, block sum of squares, fp16((x w) alpha))
template <int XV, bool NORM>
__device__ __forceinline__ void stage_input(const uint16_t *x, const float *nw, uint32_t K, float eps, u32x4 *xs,
                                            float *red)
{
    const uint32_t tid = threadIdx.x, nvec = K / 8;
    u32x4 xr[XV];
    float4 nv[NORM ? XV : 1][2];
#pragma unroll
    for (int i = 0; i < XV; ++i)
    {
        const uint32_t vi = min(tid + 256 * i, nvec - 1);
        xr[i] = ((const u32x4 *)x)[vi];
        if constexpr (NORM)
        {
            nv[i][0] = ((const float4 *)nw)[2 * vi];
            nv[i][1] = ((const float4 *)nw)[2 * vi + 1];
        }
    }
#pragma unroll
    for (int i = 0; i < XV; ++i)
        if (tid + 256 * i >= nvec)
            xr[i] = (u32x4){0, 0, 0, 0};
    if constexpr (NORM)
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
        const float alpha = 1.0f / sqrtf(ss / (float)K + eps);
#pragma unroll
        for (int i = 0; i < XV; ++i)
        {
            const float ws[8] = {nv[i][0].x, nv[i][0].y, nv[i][0].z, nv[i][0].w,
                                 nv[i][1].x, nv[i][1].y, nv[i][1].z, nv[i][1].w};
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
}

// The wave's units u = gw, gw + W, ... of a phase with `units` units of R rows (NV vectors per lane and row). On
// entry w holds unit gw's weights and e its epilogue inputs; each unit's successor is requested before the unit's
// reduction. load(u) requests unit u (weights into w, epilogue inputs into e); epi(u, acc, e) stores its outputs.
template <int R, int NV, int WN, typename Load, typename Epi>
__device__ __forceinline__ void run_units(u32x4 (&w)[WN], float (&e)[2], uint32_t units, uint32_t nvec,
                                          const u32x4 *xs, Load load, Epi epi)
{
    const uint32_t lane = threadIdx.x & 63, W = gridDim.x * 4;
    for (uint32_t u = blockIdx.x * 4 + (threadIdx.x >> 6); u < units; u += W)
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
                    acc[k] = dot8(w[k * NV + i], xv, acc[k]);
            }
        }
        const float ec[2] = {e[0], e[1]};
        if (u + W < units)
            load(u + W);
#pragma unroll
        for (int k = 0; k < R; ++k)
            acc[k] = wave_sum_dpp(acc[k]);
        if (lane == 0)
            epi(u, acc, ec);
    }
}

// fp16 to an agent-scope (written-through) 16-bit store
__device__ __forceinline__ void store_half(uint16_t *p, float v)
{
    __hip_atomic_store(p, f2h(v), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

} // namespace

// One wave per SIMD (a workgroup of 4 waves per CU) at the 7B and 13B widths: the phases' weights, input rows and the
// attention's registers, all in one kernel, take more than the 256 registers two waves per SIMD would leave.
template <int NVD, int NVF> __global__ __launch_bounds__(256, 1) void decode_persist_kernel(PersistArgs a)
{
    constexpr int WN = 2 * NVD > NVF ? 2 * NVD : NVF;
    constexpr int XD = (NVD * 64 + 255) / 256, XF = (NVF * 64 + 255) / 256; // input vectors per thread
    extern __shared__ u32x4 xs[];
    __shared__ float red[8];
    const uint32_t tid = threadIdx.x;
    const uint32_t gw = blockIdx.x * 4 + (tid >> 6);
    const uint32_t D = a.D, F = a.F, hd = a.hd, nd = D / 8, nf = F / 8;
    const uint32_t pos = a.step->offset;
    u32x4 w[WN];
    float e[2] = {0.f, 0.f};

    // unit loaders (weights of the unit's rows, and the epilogue inputs the unit's stores need)
    auto load_qkv = [&](const PersistLayer &ly, uint32_t u) {
        load_row<NVD, 0>(w, ly.wqkv, 2 * u, nd);
        load_row<NVD, NVD>(w, ly.wqkv, 2 * u + 1, nd);
        e[0] = a.freqs[((2 * u) % D) % hd / 2];
    };
    auto load_wo = [&](const PersistLayer &ly, const uint16_t *resid, uint32_t u) {
        load_row<NVD, 0>(w, ly.wo, 2 * u, nd);
        load_row<NVD, NVD>(w, ly.wo, 2 * u + 1, nd);
        e[0] = h2f(resid[2 * u]);
        e[1] = h2f(resid[2 * u + 1]);
    };
    auto load_gu = [&](const PersistLayer &ly, uint32_t u) {
        load_row<NVD, 0>(w, ly.wug, u, nd);         // up
        load_row<NVD, NVD>(w, ly.wug, F + u, nd);   // gate
    };
    auto load_down = [&](const PersistLayer &ly, const uint16_t *resid, uint32_t u) {
        load_row<NVF, 0>(w, ly.wd, u, nf);
        e[0] = h2f(resid[u]);
    };
    auto load_logits = [&](uint32_t u) { load_row<NVD, 0>(w, a.out_w, u, nd); };

    if (gw < 3 * D / 2)
        load_qkv(a.layers[0], gw);
    for (uint32_t l = 0; l < a.L; ++l)
    {
        const PersistLayer ly = a.layers[l];
        const uint16_t *h_in = a.hs + (size_t)(2 * l) * a.hstride;
        uint16_t *h_mid = a.hs + (size_t)(2 * l + 1) * a.hstride, *h_out = a.hs + (size_t)(2 * l + 2) * a.hstride;
        uint16_t *q = a.qs + (size_t)l * a.hstride, *att = a.attns + (size_t)l * a.hstride;
        uint16_t *act = a.acts + (size_t)l * a.fstride;
        const uint32_t k0 = 5 * l; // this layer's first barrier

        // A: QKV, RoPE on q and k, the position's cache rows
        if (l > 0)
            wait_barrier(a, k0 - 1);
        stage_input<XD, true>(h_in, ly.attn_norm, D, a.eps, xs, red);
        run_units<2, NVD>(w, e, 3 * D / 2, nd, xs, [&](uint32_t u) { load_qkv(ly, u); },
                          [&](uint32_t u, const float *acc, const float *ec) {
                              const uint32_t r0 = 2 * u, region = r0 / D, rr = r0 % D, head = rr / hd,
                                             dim = rr % hd;
                              const float v0 = h2f(f2h(acc[0])), v1 = h2f(f2h(acc[1]));
                              const size_t cache = ((size_t)head * a.ctx + pos) * hd + dim;
                              if (region == 2)
                              {
                                  store_pair<true>(ly.vc + cache, v0, v1);
                                  return;
                              }
                              const float f = (float)pos / ec[0];
                              const float c = cosf(f), sn = sinf(f);
                              store_pair<true>(region == 0 ? q + rr : ly.kc + cache, rope_mul_sub(c, v0, sn, v1),
                                               rope_mul_add(sn, v0, c, v1));
                          });
        finish_phase(a, k0);

        // B: attention; the Wo units' weights are requested behind the first cache reads
        wait_barrier(a, k0);
        {
            auto prefetch_wo = [&]() {
                if (gw < D / 2)
                    load_wo(ly, h_in, gw);
            };
            AttnDecodeArgs at{};
            at.q = q;
            at.kc = ly.kc;
            at.vc = ly.vc;
            at.out = att;
            at.step = a.step;
            at.H = a.H;
            at.hd = hd;
            at.ctx = a.ctx;
            at.groups = 0;
            at.scale = a.scale;
            at.small_max = a.small_max;
            // dim slices per head: the largest divisor of hd / 8 (at most 16) whose blocks fit the grid
            const uint32_t vpr = hd / 8, hb = (a.H + 7) / 8;
            uint32_t G = 1;
            for (uint32_t g = 1; g <= 16 && g <= vpr; ++g)
                if (vpr % g == 0 && 8 * g * hb <= gridDim.x)
                    G = g;
            at.groups = G;
            const uint32_t nb = 8 * G * hb;
            float *sm = (float *)xs, *part = sm + a.small_max;
            bool issued = false;
            if (pos + 1 > a.small_max)
            {
                if (tid == 0)
                    __hip_atomic_store(a.err, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
            }
            else
                for (uint32_t b = blockIdx.x; b < nb; b += gridDim.x)
                {
                    uint32_t h, g;
                    block_head(b, G, h, g);
                    if (h < a.H)
                    {
                        if (!issued)
                            small_block<256, true>(at, h, g, sm, part, prefetch_wo);
                        else
                            small_block<256, true>(at, h, g, sm, part);
                        issued = true;
                    }
                    __syncthreads();
                }
            if (!issued)
                prefetch_wo();
        }
        finish_phase(a, k0 + 1);

        // C: h' = h + Wo attn
        wait_barrier(a, k0 + 1);
        stage_input<XD, false>(att, nullptr, D, a.eps, xs, red);
        run_units<2, NVD>(w, e, D / 2, nd, xs, [&](uint32_t u) { load_wo(ly, h_in, u); },
                          [&](uint32_t u, const float *acc, const float *ec) {
                              store_pair<true>(h_mid + 2 * u, ec[0] + h2f(f2h(acc[0])), ec[1] + h2f(f2h(acc[1])));
                          });
        finish_phase(a, k0 + 2);
        if (gw < F)
            load_gu(ly, gw);

        // D: up * silu(gate) of RMSNorm(h')
        wait_barrier(a, k0 + 2);
        stage_input<XD, true>(h_mid, ly.ffn_norm, D, a.eps, xs, red);
        run_units<2, NVD>(w, e, F, nd, xs, [&](uint32_t u) { load_gu(ly, u); },
                          [&](uint32_t u, const float *acc, const float *) {
                              const float up = h2f(f2h(acc[0]));
                              const float gate = h2f(f2h(silu(acc[1])));
                              store_half(act + u, up * gate);
                          });
        finish_phase(a, k0 + 3);
        if (gw < D)
            load_down(ly, h_mid, gw);

        // E: h'' = h' + Wd act
        wait_barrier(a, k0 + 3);
        stage_input<XF, false>(act, nullptr, F, a.eps, xs, red);
        run_units<1, NVF>(w, e, D, nf, xs, [&](uint32_t u) { load_down(ly, h_mid, u); },
                          [&](uint32_t u, const float *acc, const float *ec) {
                              store_half(h_out + u, ec[0] + h2f(f2h(acc[0])));
                          });
        finish_phase(a, k0 + 4);
        if (l + 1 < a.L)
        {
            if (gw < 3 * D / 2)
                load_qkv(a.layers[l + 1], gw);
        }
        else if (gw < a.V)
            load_logits(gw);
    }

    // the output norm, the vocabulary product and its arg max (lane 0 keeps the best of the rows it stores)
    wait_barrier(a, 5 * a.L - 1);
    stage_input<XD, true>(a.hs + (size_t)(2 * a.L) * a.hstride, a.out_norm, D, a.eps, xs, red);
    float bv = -INFINITY;
    uint32_t bi = 0xFFFFFFFFu;
    run_units<1, NVD>(w, e, a.V, nd, xs, [&](uint32_t u) { load_logits(u); },
                      [&](uint32_t u, const float *acc, const float *) {
                          a.logits[u] = f2h(acc[0]);
                          const float v = h2f(f2h(acc[0]));
                          if (am_before(v, u, bv, bi))
                          {
                              bv = v;
                              bi = u;
                          }
                      });
    GemvArgs g{};
    g.am_ids = a.am_ids;
    g.am_io = a.am_io;
    g.am_val = a.am_val;
    g.am_idx = a.am_idx;
    g.am_count = a.am_count;
    gemv_argmax_finish(g, bv, bi);

    // every workgroup has passed its last wait once all of them are here: clear the words for the next launch
    __syncthreads();
    if (tid == 0 &&
        __hip_atomic_fetch_add(a.sync + kPDone, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == gridDim.x - 1)
    {
        for (uint32_t c = 0; c < 8; ++c)
            __hip_atomic_store(a.sync + kPStride * c, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(a.sync + kPTop, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(a.sync + kPFlag, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(a.sync + kPAbort, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(a.sync + kPDone, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}

// ---------------------------------------------------------------------------------------------------------------

template <int NVD, int NVF> static hipError_t launch_persist_nv(hipStream_t st, const PersistArgs &a, int cu_count)
{
    // LDS: the largest input row, or the attention's scores and partial sums
    const size_t lds = std::max({(size_t)a.D * 2, (size_t)a.F * 2, ((size_t)a.small_max + 4 * a.hd) * sizeof(float)});
    static uint64_t occ_memo = 0;
    const int per_cu = occupancy_per_cu((const void *)decode_persist_kernel<NVD, NVF>, 256, lds, occ_memo);
    if (per_cu < 1)
        return hipErrorInvalidConfiguration;
    // every workgroup waits for all the others: the grid is what the device holds at once (at most 2 per CU)
    const uint32_t grid = (uint32_t)(cu_count > 0 ? cu_count : 256) * (uint32_t)std::min(per_cu, 2);
    if (grid > a.am_cap)
        return hipErrorInvalidValue;
    // the attention part: the slices the kernel picks, and the V rows its 256-thread blocks cover
    const uint32_t vpr = a.hd / 8, hb = (a.H + 7) / 8;
    uint32_t G = 1;
    for (uint32_t g = 1; g <= 16 && g <= vpr; ++g)
        if (vpr % g == 0 && 8 * g * hb <= grid)
            G = g;
    const uint32_t lpr = vpr / G, seg = 64 / lpr, rpp = 4 * seg;
    if (lpr > 4 || 64 % lpr != 0 || (uint64_t)a.small_max > (uint64_t)kSmallMaxPasses * rpp)
        return hipErrorInvalidValue;
    decode_persist_kernel<NVD, NVF><<<grid, 256, lds, st>>>(a);
    return hipGetLastError();
}

hipError_t launch_decode_persist(hipStream_t st, const PersistArgs &a, int cu_count)
{
    if (!a.layers || a.L == 0 || a.D == 0 || a.D % 8 != 0 || a.F % 8 != 0 || a.F == 0 || a.hd == 0 ||
        a.hd % 8 != 0 || a.hd > 256 || a.H * a.hd != a.D || a.V == 0 || a.small_max == 0 || a.small_max > a.ctx ||
        a.hstride % 128 != 0 || a.hstride < a.D || a.fstride % 128 != 0 || a.fstride < a.F || !a.hs || !a.qs ||
        !a.attns || !a.acts || !a.logits || !a.sync || !a.err || !a.am_ids || !a.am_val || !a.am_idx || !a.am_count)
        return hipErrorInvalidValue;
    const uint32_t nvd = (a.D / 8 + 63) / 64, nvf = (a.F / 8 + 63) / 64;
#define PERSIST_CASE(NVD_, NVF_)                                                                                    \
    if (nvd == NVD_ && nvf == NVF_)                                                                                 \
        return launch_persist_nv<NVD_, NVF_>(st, a, cu_count);
    PERSIST_CASE(1, 1) // small shapes: dim up to 512, FFN up to 512 (or 1024)
    PERSIST_CASE(1, 2)
    PERSIST_CASE(8, 22)  // LLaMA-2-7B: dim 4096, FFN 11008
    PERSIST_CASE(10, 27) // LLaMA-2-13B: dim 5120, FFN 13824
#undef PERSIST_CASE
    return hipErrorInvalidValue;
}

} // namespace vk
