// Prompt-step weight products of at most 128 tokens with the weights streamed as matrix-core fragments:
// C[M, N] = X[M, K] . W[N, K]^T, M <= 128, fp16 operands and fp32 accumulation. Takes the place of
// src/shaders/vkllm_matmul_t1.comp for the short-prompt token step, where a product is bound by reading its weights
// once.
//
// Layouts. The weights are read from a fragment-tiled copy: 1 KB blocks, each the A operand of one
// v_mfma_f32_32x32x16_f16. Block (rb, ks) (at (rb * K / 16 + ks) KB) holds rows 32 rb .. 32 rb + 31 and columns
// 16 ks .. 16 ks + 15, lane l's 16 bytes being row 32 rb + l % 32, columns 16 ks + 8 (l / 32) .. + 7, so a wave
// fetches an operand with one contiguous 1 KB load. (Streaming reads of 180 MB on MI355X: 6.35 TB/s as contiguous
// 1 KB loads, 4.0-4.3 TB/s as 16 row-major rows of 64 bytes per load, 2.4 TB/s as 32 rows of 32 bytes.) Rows past N
// are zero. The FFN's [Wu; Wg] is tiled with its rows interleaved: block rb holds up rows 16 rb .. 16 rb + 15, then
// gate rows 16 rb .. 16 rb + 15, so both values of an output column meet in one lane. X is fragment-ordered
// (xt_vec), as the RMSNorm, residual-norm and attention kernels write it for these products.
//
// Kernel. A workgroup has CW compute waves and one loader wave. Compute wave w owns row block rb and streams its
// fragments straight into registers 16 K steps ahead; a K step is MB MFMAs (32 rows x 32 tokens each), with the next
// step's B operands read from LDS during them. The loader copies X through three LDS buffers of 8 K steps (MB KB
// each); it writes a chunk two chunks ahead of the compute and requests the next one as it does, so its loads have
// two chunks of compute to arrive. The waves meet at one barrier per chunk whose fences order only LDS, so the
// weight loads stay in flight across it. Split K (STREAM_PARTIAL) gives products with few row blocks enough
// workgroups; their fp32 partials go through the split-K reduce of gemm_mfma.hip. The QKV product splits the tokens
// instead (two workgroups per row group, 64 tokens each, on one XCD one after the other, so the second reads the
// weights from L2): no partials, and RoPE with the K/V append runs in its epilogue.
#include <utility>

#include "device_common.h"
#include "kernels.h"

namespace vk
{

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int kStreamAhead = 16; // weight K steps in flight per compute wave
constexpr int kStreamChunk = 8;  // K steps per LDS chunk of X
constexpr int kStreamBufs = 3;   // LDS chunk buffers

template <int... J, typename F> __device__ __forceinline__ void stream_seq(std::integer_sequence<int, J...>, F &&f)
{
    (f(std::integral_constant<int, J>{}), ...);
}

// workgroup barrier that orders LDS only: the fences wait for the wave's LDS operations, not its global loads
__device__ __forceinline__ void lds_barrier()
{
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// one 16-byte vector of the tiled copy per thread (grid-stride): vector v is lane v % 64 of block v / 64
__global__ __launch_bounds__(256) void tile_weights_kernel(const uint16_t *W, uint16_t *Wt, uint32_t N, uint32_t K,
                                                           uint32_t F, uint64_t total)
{
    const uint32_t KS = K / 16;
    for (uint64_t v = (uint64_t)blockIdx.x * 256 + threadIdx.x; v < total; v += (uint64_t)gridDim.x * 256)
    {
        const uint32_t lane = (uint32_t)(v % 64), i = lane % 32;
        const uint64_t blk = v / 64;
        const uint32_t ks = (uint32_t)(blk % KS), rb = (uint32_t)(blk / KS);
        uint32_t row = rb * 32 + i;
        bool ok = row < N;
        if (F)
        {
            row = i < 16 ? 16 * rb + i : F + 16 * rb + i - 16;
            ok = true;
        }
        u32x4 val = {0u, 0u, 0u, 0u};
        if (ok)
            val = *(const u32x4 *)(W + (size_t)row * K + ks * 16 + (lane / 32) * 8);
        ((u32x4 *)Wt)[v] = val;
    }
}

size_t stream_tiled_elems(uint32_t N, uint32_t K, uint32_t F)
{
    return (size_t)(F ? 2 * F : (N + 31) / 32 * 32) * K;
}

hipError_t launch_tile_weights(hipStream_t st, const uint16_t *W, uint16_t *Wt, uint32_t N, uint32_t K, uint32_t F)
{
    if (K == 0 || K % 16 != 0 || N == 0 || (F && (N != 2 * F || F % 16 != 0)))
        return hipErrorInvalidValue;
    const uint64_t total = stream_tiled_elems(N, K, F) / 8;
    const uint64_t blocks = (total + 255) / 256;
    tile_weights_kernel<<<(uint32_t)(blocks < 8192 ? blocks : 8192), 256, 0, st>>>(W, Wt, N, K, F, total);
    return hipGetLastError();
}

// row-major X [M, K] -> fragment order (xt_vec), rows M..127 zero; one 16-byte vector per thread (grid-stride)
__global__ __launch_bounds__(256) void tile_activations_kernel(const uint16_t *X, uint16_t *Xt, uint32_t M, uint32_t K)
{
    const uint32_t total = 128 * K / 8;
    for (uint32_t v = blockIdx.x * 256 + threadIdx.x; v < total; v += gridDim.x * 256)
    {
        // v = (kv / 2 * 4 + t / 32) * 64 + (kv % 2) * 32 + t % 32
        const uint32_t lane = v % 64, t = (v / 64) % 4 * 32 + lane % 32, kv = v / 256 * 2 + lane / 32;
        u32x4 val = {0u, 0u, 0u, 0u};
        if (t < M)
            val = *(const u32x4 *)(X + (size_t)t * K + kv * 8);
        ((u32x4 *)Xt)[v] = val;
    }
}

hipError_t launch_tile_activations(hipStream_t st, const uint16_t *X, uint16_t *Xt, uint32_t M, uint32_t K)
{
    if (M == 0 || M > 128 || K == 0 || K % 16 != 0)
        return hipErrorInvalidValue;
    const uint32_t blocks = (128 * K / 8 + 255) / 256;
    tile_activations_kernel<<<blocks < 4096 ? blocks : 4096, 256, 0, st>>>(X, Xt, M, K);
    return hipGetLastError();
}

// STREAM_QKV_ROPE: columns n .. n + 3 (n % 4 == 0) of token t, fp16-rounded as the split-K reduce rounds them: two
// RoPE pairs of q or k rotated and stored, or four v values stored, as one 8-byte vector (rope_store8's arithmetic)
__device__ __forceinline__ void rope_store4(const GemmRope &r, uint32_t t, uint32_t n, float a0, float a1, float a2,
                                            float a3)
{
    const uint32_t region = (n >= r.D) + (n >= 2 * r.D), c = n - region * r.D, head = c / r.hd, dim = c % r.hd;
    const float v0 = h2f(f2h(a0)), v1 = h2f(f2h(a1)), v2 = h2f(f2h(a2)), v3 = h2f(f2h(a3));
    const size_t cache = ((size_t)head * r.ctx + r.offset + t) * r.hd + dim;
    if (region == 2)
    {
        *(uint2 *)(r.vc + cache) = uint2{pack2(f2h(v0), f2h(v1)), pack2(f2h(v2), f2h(v3))};
        return;
    }
    const float *cs = r.cs + ((size_t)t * (r.hd / 2) + dim / 2) * 2;
    const uint2 o = {pack2(f2h(rope_mul_sub(cs[0], v0, cs[1], v1)), f2h(rope_mul_add(cs[1], v0, cs[0], v1))),
                     pack2(f2h(rope_mul_sub(cs[2], v2, cs[3], v3)), f2h(rope_mul_add(cs[3], v2, cs[2], v3)))};
    *(uint2 *)(region == 0 ? r.q + (size_t)t * r.D + c : r.kc + cache) = o;
}

// MS token parts: workgroup L takes row group g and token blocks [tb0, tb0 + MB). With MS > 1 the parts of a row
// group get consecutive slots of one XCD (workgroups are dealt to the 8 XCDs round robin).
template <int EPI, int MB, int CW, int MS>
__global__ __launch_bounds__((CW + 1) * 64, 1) void stream_gemm_kernel(const uint16_t *__restrict__ X,
                                                                       const uint16_t *__restrict__ Wt, uint16_t *C,
                                                                       float *work, uint32_t M, uint32_t N,
                                                                       uint32_t K, uint32_t ldc, uint32_t kchunk,
                                                                       GemmRope rope)
{
    constexpr int U = kStreamAhead, KSC = kStreamChunk, NB = kStreamBufs;
    constexpr int BUFV = KSC * MB * 64; // 16-byte vectors per LDS buffer
    static_assert(U % KSC == 0, "the weight ring spans whole chunks");
    extern __shared__ u32x4 xs[];
    const uint32_t lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const uint32_t nrb = (N + 31) / 32;
    uint32_t g = blockIdx.x, tb0 = 0;
    if constexpr (MS > 1)
    {
        const uint32_t slot = blockIdx.x / 8;
        g = (slot / MS) * 8 + blockIdx.x % 8;
        tb0 = (slot % MS) * MB;
        if (g * CW >= nrb)
            return; // padding of the last XCD round (whole workgroup, before any barrier)
    }
    const uint32_t kb = blockIdx.y * kchunk, ke = min(K, kb + kchunk);
    if (kb >= ke)
        return; // whole workgroup (the launcher sizes the splits so that none is empty)
    const uint32_t ks0 = kb / 16, nks = (ke - kb) / 16, nch = (nks + KSC - 1) / KSC;

    if (w == CW)
    {
        // loader: chunk c into buffer c % NB. Chunks 0 and 1 before barrier 0; after barrier c it writes chunk c + 2
        // (requested after barrier c - 1) and requests chunk c + 3. Steps past the range re-read the last one.
        const u32x4 *xp = (const u32x4 *)X + lane;
        u32x4 r[KSC * MB];
        auto issue = [&](uint32_t c) {
#pragma unroll
            for (int j = 0; j < KSC; ++j)
            {
                const uint32_t ks = ks0 + min(c * KSC + j, nks - 1);
#pragma unroll
                for (int tb = 0; tb < MB; ++tb)
                    r[j * MB + tb] = xp[(size_t)(ks * 4 + tb0 + tb) * 64];
            }
        };
        auto write = [&](uint32_t c) {
            u32x4 *b = xs + (c % NB) * BUFV + lane;
#pragma unroll
            for (int i = 0; i < KSC * MB; ++i)
                b[i * 64] = r[i];
        };
        for (uint32_t c = 0; c < 2 && c < nch; ++c)
        {
            issue(c);
            write(c);
        }
        if (2 < nch)
            issue(2);
        for (uint32_t c = 0; c < nch; ++c)
        {
            lds_barrier();
            if (c + 2 < nch)
                write(c + 2);
            if (c + 3 < nch)
                issue(c + 3);
        }
        return;
    }

    const uint32_t rbw = g * CW + w, rb = min(rbw, nrb - 1);
    const u32x4 *wp = (const u32x4 *)Wt + ((size_t)rb * (K / 16) + ks0) * 64 + lane;
    f32x16 acc[MB];
#pragma unroll
    for (int tb = 0; tb < MB; ++tb)
#pragma unroll
        for (int e = 0; e < 16; ++e)
            acc[tb][e] = 0.f;
    u32x4 wf[U];
#pragma unroll
    for (int i = 0; i < U; ++i)
        wf[i] = __builtin_nontemporal_load(wp + (size_t)min((uint32_t)i, nks - 1) * 64);
    u32x4 bf[2][MB];
    // B operands of step s; the next chunk is complete once the current one's barrier has passed (three buffers)
    auto readb = [&](uint32_t s, int into) {
        const u32x4 *b = xs + ((s / KSC) % NB) * BUFV + (s % KSC) * MB * 64 + lane;
#pragma unroll
        for (int tb = 0; tb < MB; ++tb)
            bf[into][tb] = b[tb * 64];
    };
    // step s with ring slot I: the next step's B reads between this step's MFMAs, then slot I refilled with step
    // s + U
    auto step = [&](auto slot, uint32_t s) {
        constexpr int I = decltype(slot)::value;
        readb(min(s + 1, nks - 1), (I + 1) & 1);
#pragma unroll
        for (int tb = 0; tb < MB; ++tb)
            acc[tb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, wf[I]),
                                                             __builtin_bit_cast(f16x8, bf[I & 1][tb]), acc[tb], 0, 0,
                                                             0);
        wf[I] = __builtin_nontemporal_load(wp + (size_t)min(s + U, nks - 1) * 64);
#pragma unroll
        for (int tb = 0; tb < MB; ++tb)
        {
            __builtin_amdgcn_sched_group_barrier(0x100, 1, 0); // LDS read
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0); // MFMA
        }
        __builtin_amdgcn_sched_group_barrier(0x020, 1, 0); // global load
    };
    lds_barrier(); // barrier 0: chunks 0 and 1 are in
    readb(0, 0);
    uint32_t s = 0;
    // one barrier per chunk boundary, as the loader's loop
    for (; s + U <= nks; s += U)
        stream_seq(std::make_integer_sequence<int, U>{}, [&](auto i) {
            constexpr int I = decltype(i)::value;
            if constexpr (I % KSC == 0)
            {
                if (I > 0 || s > 0)
                    lds_barrier();
            }
            step(i, s + I);
        });
    stream_seq(std::make_integer_sequence<int, U>{}, [&](auto i) {
        constexpr int I = decltype(i)::value;
        if (s + I < nks)
        {
            if (I % KSC == 0 && s + I > 0)
                lds_barrier();
            step(i, s + I);
        }
    });
    if (rbw >= nrb)
        return;

    // acc[tb][r] is row 32 rb + (r / 4) * 8 + (lane / 32) * 4 + r % 4 of token 32 tb + lane % 32
#pragma unroll
    for (int tb = 0; tb < MB; ++tb)
    {
        const uint32_t t = (tb0 + tb) * 32 + lane % 32;
        if (t >= M)
            continue;
        if constexpr (EPI == STREAM_QKV_ROPE)
        {
#pragma unroll
            for (int q = 0; q < 4; ++q)
                rope_store4(rope, t, rb * 32 + q * 8 + (lane / 32) * 4, acc[tb][q * 4], acc[tb][q * 4 + 1],
                            acc[tb][q * 4 + 2], acc[tb][q * 4 + 3]);
        }
        else if constexpr (EPI == STREAM_SWIGLU)
        {
            // rows r < 8 are up rows u = (r / 4) * 8 + (lane / 32) * 4 + r % 4 of output block rb, r + 8 their gate
#pragma unroll
            for (int h = 0; h < 2; ++h)
            {
                const uint32_t u = h * 8 + (lane / 32) * 4;
                const uint2 o = {pack2(swiglu_out(acc[tb][h * 4], acc[tb][8 + h * 4]),
                                       swiglu_out(acc[tb][h * 4 + 1], acc[tb][9 + h * 4])),
                                 pack2(swiglu_out(acc[tb][h * 4 + 2], acc[tb][10 + h * 4]),
                                       swiglu_out(acc[tb][h * 4 + 3], acc[tb][11 + h * 4]))};
                *(uint2 *)(C + (size_t)t * ldc + rb * 16 + u) = o;
            }
        }
        else
        {
#pragma unroll
            for (int g = 0; g < 4; ++g)
            {
                const uint32_t n = rb * 32 + g * 8 + (lane / 32) * 4;
                if constexpr (EPI == STREAM_PARTIAL)
                    *(f32x4 *)(work + ((size_t)blockIdx.y * M + t) * N + n) =
                        f32x4{acc[tb][g * 4], acc[tb][g * 4 + 1], acc[tb][g * 4 + 2], acc[tb][g * 4 + 3]};
                else if (n + 3 < N)
                    *(uint2 *)(C + (size_t)t * ldc + n) = uint2{pack2(f2h(acc[tb][g * 4]), f2h(acc[tb][g * 4 + 1])),
                                                                pack2(f2h(acc[tb][g * 4 + 2]), f2h(acc[tb][g * 4 + 3]))};
                else
                {
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        if (n + e < N)
                            C[(size_t)t * ldc + n + e] = f2h(acc[tb][g * 4 + e]);
                }
            }
        }
    }
}

template <int EPI, int MB, int CW, int MS = 1>
static hipError_t launch_stream_shape(hipStream_t st, const uint16_t *X, const uint16_t *Wt, uint16_t *C, float *work,
                                      uint32_t M, uint32_t N, uint32_t K, uint32_t ldc, uint32_t kchunk, dim3 grid,
                                      const GemmRope &rope = GemmRope{})
{
    static uint64_t attr_devs = 0; // devices on which the LDS limit is raised for this kernel
    constexpr size_t lds = (size_t)kStreamBufs * kStreamChunk * MB * 1024;
    hipError_t e = lds_attr_once((const void *)stream_gemm_kernel<EPI, MB, CW, MS>, lds, attr_devs);
    if (e != hipSuccess)
        return e;
    stream_gemm_kernel<EPI, MB, CW, MS><<<grid, (CW + 1) * 64, lds, st>>>(X, Wt, C, work, M, N, K, ldc, kchunk, rope);
    return hipGetLastError();
}

template <int EPI, int CW>
static hipError_t launch_stream_mb(hipStream_t st, const uint16_t *X, const uint16_t *Wt, uint16_t *C, float *work,
                                   uint32_t M, uint32_t N, uint32_t K, uint32_t ldc, uint32_t kchunk, dim3 grid)
{
    switch ((M + 31) / 32)
    {
    case 1:
        return launch_stream_shape<EPI, 1, CW>(st, X, Wt, C, work, M, N, K, ldc, kchunk, grid);
    case 2:
        return launch_stream_shape<EPI, 2, CW>(st, X, Wt, C, work, M, N, K, ldc, kchunk, grid);
    case 3:
        return launch_stream_shape<EPI, 3, CW>(st, X, Wt, C, work, M, N, K, ldc, kchunk, grid);
    default:
        return launch_stream_shape<EPI, 4, CW>(st, X, Wt, C, work, M, N, K, ldc, kchunk, grid);
    }
}

// [Wq; Wk; Wv] with RoPE: three compute waves per workgroup; above 32 tokens two token parts (256 workgroups at the
// 7B widths: at 128 tokens the same time as two K ranges, with no partials to add)
static hipError_t launch_stream_qkv(hipStream_t st, const uint16_t *X, const uint16_t *Wt, uint32_t M, uint32_t N,
                                    uint32_t K, const GemmRope &r)
{
    if (!r.q || !r.kc || !r.vc || !r.cs || r.D == 0 || r.D % 32 != 0 || N != 3 * r.D || r.hd < 4 || r.hd % 4 != 0 ||
        r.D % r.hd != 0 || r.offset + M > r.ctx)
        return hipErrorInvalidValue;
    const uint32_t groups = ((N + 31) / 32 + 2) / 3;
    const dim3 split_grid((groups + 7) / 8 * 8 * 2, 1);
    if (M > 64)
        return launch_stream_shape<STREAM_QKV_ROPE, 2, 3, 2>(st, X, Wt, nullptr, nullptr, M, N, K, 0, K, split_grid, r);
    if (M > 32)
        return launch_stream_shape<STREAM_QKV_ROPE, 1, 3, 2>(st, X, Wt, nullptr, nullptr, M, N, K, 0, K, split_grid, r);
    return launch_stream_shape<STREAM_QKV_ROPE, 1, 3>(st, X, Wt, nullptr, nullptr, M, N, K, 0, K, dim3(groups, 1), r);
}

hipError_t launch_stream_gemm(hipStream_t st, int epi, const uint16_t *X, const uint16_t *Wt, uint16_t *C,
                              float *work, size_t work_elems, uint32_t M, uint32_t N, uint32_t K, uint32_t ldc,
                              uint32_t *splits, const GemmRope *rope)
{
    if (M == 0 || M > 128 || N == 0 || K == 0 || K % 16 != 0 || !splits)
        return hipErrorInvalidValue;
    if (epi == STREAM_QKV_ROPE)
    {
        if (!rope)
            return hipErrorInvalidValue;
        *splits = 1;
        return launch_stream_qkv(st, X, Wt, M, N, K, *rope);
    }
    const uint32_t nrb = (N + 31) / 32, chunks = (K / 16 + kStreamChunk - 1) / kStreamChunk;
    // three compute waves for the SwiGLU product when that still fits one workgroup per CU (more CUs take part)
    const uint32_t cw = epi == STREAM_SWIGLU && (nrb + 2) / 3 <= 256 ? 3 : 4;
    const uint32_t groups = (nrb + cw - 1) / cw;
    uint32_t n_splits = 1, kchunk = K;
    if (epi == STREAM_PARTIAL)
    {
        if (N % 32 != 0 || !work)
            return hipErrorInvalidValue;
        // about three workgroups for every four CUs: split K when the row blocks alone leave most CUs idle (7B Wo at
        // 128 tokens: 6 K ranges, 192 workgroups, 15.2 us against 16.7 us for 8 ranges; fewer partials to add)
        uint32_t want = *splits ? *splits : 192 / groups;
        want = want < 1 ? 1 : (want > 8 ? 8 : want);
        want = want > chunks ? chunks : want;
        const uint32_t per = (chunks + want - 1) / want;
        n_splits = (chunks + per - 1) / per;
        kchunk = per * kStreamChunk * 16;
        if ((size_t)n_splits * M * N > work_elems)
            return hipErrorInvalidValue;
    }
    else if (epi == STREAM_SWIGLU)
    {
        if (N % 32 != 0 || ldc < N / 2)
            return hipErrorInvalidValue;
    }
    else if (epi != STREAM_PLAIN || ldc < N || ldc % 4 != 0 || (uintptr_t)C % 8 != 0)
        return hipErrorInvalidValue; // the plain store writes 4 outputs of a row as one 8-byte vector
    *splits = n_splits;
    const dim3 grid(groups, n_splits);
    switch (epi)
    {
    case STREAM_PARTIAL:
        return launch_stream_mb<STREAM_PARTIAL, 4>(st, X, Wt, C, work, M, N, K, ldc, kchunk, grid);
    case STREAM_PLAIN:
        return launch_stream_mb<STREAM_PLAIN, 4>(st, X, Wt, C, work, M, N, K, ldc, kchunk, grid);
    default:
        if (cw == 3)
            return launch_stream_mb<STREAM_SWIGLU, 3>(st, X, Wt, C, work, M, N, K, ldc, kchunk, grid);
        return launch_stream_mb<STREAM_SWIGLU, 4>(st, X, Wt, C, work, M, N, K, ldc, kchunk, grid);
    }
}

} // namespace vk
