// Prefill GEMM on CDNA4 matrix cores: C[M, N] = A[M, K] . B[N, K]^T with fp16 operands and fp32 accumulation.
// It replaces src/shaders/vkllm_matmul_t1.comp for the token step's weight products, where A holds the step's
// activations (M = tokens) and B a weight matrix stored [out, in].
//
// gemm32_kernel (K a multiple of 64, every prefill product of the LLaMA-2 shapes): v_mfma_f32_32x32x16_f16 on
// 256 x 256 or 128 x 128 tiles of 256-thread workgroups, 2 x 2 waves each owning a (BM/2) x (BN/2) grid of 32x32
// blocks (up to 256 fp32 accumulators per lane), K in steps of 64 through two LDS buffers with rows padded to 144
// bytes (the operand reads of 8 lanes then fall on distinct banks). A step is straight-line code whose instruction
// stream group barriers lay out as MFMAs with, between them, the next 16-wide slice's operand reads, the next
// step's global loads (first slice) and their stores into the other LDS buffer (last slice), so memory traffic
// runs under the matrix pipe; one barrier per step. Its epilogue stages the tile's fp16 outputs in the freed LDS and
// stores 16-byte row chunks: plain, SiLU on columns >= split, residual add, the FFN's SwiGLU (reading [Wu; Wg] as
// interleaved 32-row blocks), or the QKV product's RoPE with q and the K/V cache rows written directly.
// gemm_kernel (other K): v_mfma_f32_16x16x32_f16, 128 x 128 or 128 x 64 tiles, the same double buffering, with the
// K tail zeroed (plain, SiLU and residual epilogues only).
//
// Narrow products split K over several workgroups; the fp32 partial tiles are added in split order by
// gemm_splitk_reduce_kernel, which applies the epilogue, or for a residual product followed by RMSNorm by
// gemm_resid_norm_kernel, which also normalises the rows. Tiles are ordered M-fastest and dealt to XCDs in
// contiguous runs so a run shares its B tiles in one L2. Global loads are unconditional at clamped addresses (a
// guarded load compiles to a branch and a wait per load).
#include <type_traits>
#include <utility>

#include "device_common.h"
#include "kernels.h"

namespace vk
{

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kBK = 64;
constexpr int kLdsRow = kBK + 8; // halfs per LDS row (144 bytes)

__device__ __forceinline__ void gemm_store(int epi, uint16_t *C, uint32_t ldc, uint32_t m, uint32_t n, float v,
                                           uint32_t split)
{
    uint16_t *c = C + (size_t)m * ldc + n;
    if (epi == GEMM_PLAIN)
        *c = f2h(v);
    else if (epi == GEMM_SILU_HI)
        *c = f2h(n >= split ? silu(v) : v);
    else
        *c = f2h(h2f(*c) + h2f(f2h(v)));
}

// GEMM_SWIGLU: product column c of [Wu; Wg] (F rows each, F % 32 == 0) is up row 32 (c / 64) + c % 32 when
// (c / 32) is even, else gate row F + 32 (c / 64) + c % 32; the output column of up column c is 32 (c / 64) + c % 32
template <int EPI> __device__ __forceinline__ uint32_t gemm_b_row(uint32_t c, uint32_t F)
{
    if constexpr (EPI == GEMM_SWIGLU)
        return 32 * (c / 64) + c % 32 + ((c / 32) % 2) * F;
    else
        return c;
}
__device__ __forceinline__ uint32_t swiglu_col(uint32_t c)
{
    return 32 * (c / 64) + c % 32;
}

// GEMM_QKV_ROPE: element (m, c) of region `region` (0 q, 1 k, 2 v) at head `head`, head dim `dim`; v is the
// element's fp16-rounded value and w its RoPE partner's (dim ^ 1), as launch_rope_kv combines them
__device__ __forceinline__ void rope_store(const GemmRope &r, uint32_t m, uint32_t region, uint32_t c,
                                           uint32_t head, uint32_t dim, float v, float w)
{
    const size_t cache = ((size_t)head * r.ctx + r.offset + m) * r.hd + dim;
    if (region == 2)
    {
        r.vc[cache] = f2h(v);
        return;
    }
    const float *cs = r.cs + ((size_t)m * (r.hd / 2) + dim / 2) * 2;
    const float out = (dim & 1) == 0 ? rope_mul_sub(cs[0], v, cs[1], w) : rope_mul_add(cs[1], w, cs[0], v);
    if (region == 0)
        r.q[(size_t)m * r.D + c] = f2h(out);
    else
        r.kc[cache] = f2h(out);
}

// GEMM_QKV_ROPE: 8 consecutive product columns from `a` (a multiple of 8) of row m, as fp16: four RoPE pairs of q
// or k rotated and stored, or v stored, as one 16-byte vector each
__device__ __forceinline__ void rope_store8(const GemmRope &r, uint32_t m, uint32_t a, u32x4 v)
{
    const uint32_t region = (a >= r.D) + (a >= 2 * r.D), c = a - region * r.D, head = c / r.hd, dim = c % r.hd;
    const size_t cache = ((size_t)head * r.ctx + r.offset + m) * r.hd + dim;
    if (region == 2)
    {
        *(u32x4 *)(r.vc + cache) = v;
        return;
    }
    const float *cs = r.cs + ((size_t)m * (r.hd / 2) + dim / 2) * 2;
    u32x4 o;
#pragma unroll
    for (int k = 0; k < 4; ++k)
    {
        const float x0 = half_lo(v[k]), x1 = half_hi(v[k]), co = cs[2 * k], sn = cs[2 * k + 1];
        o[k] = pack2(f2h(rope_mul_sub(co, x0, sn, x1)), f2h(rope_mul_add(sn, x0, co, x1)));
    }
    *(u32x4 *)(region == 0 ? r.q + (size_t)m * r.D + c : r.kc + cache) = o;
}

// SPLIT: workgroup z of gridDim.y covers K columns [z * kchunk, min(K, (z + 1) * kchunk)) and writes its fp32 tile
// to work[z][M][N] instead of C
template <int BM, int BN, int EPI, bool SPLIT>
__global__ __launch_bounds__(256) void gemm_kernel(const uint16_t *__restrict__ A, const uint16_t *__restrict__ B,
                                                   uint16_t *C, float *work, uint32_t M, uint32_t N, uint32_t K,
                                                   uint32_t ldc, uint32_t split, uint32_t kchunk, uint32_t tiles_m,
                                                   uint32_t tiles_total)
{
    constexpr int TM = BM / 32, TN = BN / 32;            // 16x16 blocks per wave
    constexpr int AV = BM * kBK / 8 / 256, BV = BN * kBK / 8 / 256; // 16-byte vectors per thread per K step
    extern __shared__ __attribute__((aligned(16))) uint16_t lds[];
    // buffer b of A at lds[b BM rows], of B after both A buffers
    auto As = [&](int b) { return lds + b * BM * kLdsRow; };
    auto Bs = [&](int b) { return lds + 2 * BM * kLdsRow + b * BN * kLdsRow; };

    const uint32_t per_xcd = gridDim.x / 8;
    const uint32_t t = (blockIdx.x % 8) * per_xcd + blockIdx.x / 8;
    if (t >= tiles_total)
        return;
    const uint32_t m0 = (t % tiles_m) * BM, n0 = (t / tiles_m) * BN;
    const uint32_t kb = SPLIT ? blockIdx.y * kchunk : 0;
    const uint32_t ke = SPLIT ? min(K, kb + kchunk) : K;
    const uint32_t tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
    const uint32_t wm = wid >> 1, wn = wid & 1;

    f32x4 acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
            acc[i][j] = (f32x4){0.f, 0.f, 0.f, 0.f};

    // rows past M or N only feed outputs that are never stored; columns past the K range are zeroed
    u32x4 ra[AV], rb[BV];
    auto load = [&](uint32_t k0) {
#pragma unroll
        for (int i = 0; i < AV; ++i)
        {
            const uint32_t v = tid + 256 * i, row = min(m0 + v / 8, M - 1), kk = k0 + (v % 8) * 8;
            const u32x4 x = *(const u32x4 *)(A + (size_t)row * K + min(kk, K - 8));
            ra[i] = kk < ke ? x : (u32x4){0, 0, 0, 0};
        }
#pragma unroll
        for (int i = 0; i < BV; ++i)
        {
            const uint32_t v = tid + 256 * i, row = min(n0 + v / 8, N - 1), kk = k0 + (v % 8) * 8;
            const u32x4 x = __builtin_nontemporal_load((const u32x4 *)(B + (size_t)row * K + min(kk, K - 8)));
            rb[i] = kk < ke ? x : (u32x4){0, 0, 0, 0};
        }
    };
    auto stash = [&](int buf) {
#pragma unroll
        for (int i = 0; i < AV; ++i)
        {
            const uint32_t v = tid + 256 * i;
            *(u32x4 *)(As(buf) + (v / 8) * kLdsRow + (v % 8) * 8) = ra[i];
        }
#pragma unroll
        for (int i = 0; i < BV; ++i)
        {
            const uint32_t v = tid + 256 * i;
            *(u32x4 *)(Bs(buf) + (v / 8) * kLdsRow + (v % 8) * 8) = rb[i];
        }
    };

    load(kb);
    stash(0);
    __syncthreads();
    int cur = 0;
    for (uint32_t k0 = kb; k0 < ke; k0 += kBK)
    {
        const bool more = k0 + kBK < ke;
        if (more)
            load(k0 + kBK);
#pragma unroll
        for (int kk = 0; kk < kBK; kk += 32)
        {
            f16x8 af[TM], bf[TN];
#pragma unroll
            for (int i = 0; i < TM; ++i)
                af[i] = *(const f16x8 *)(As(cur) + (wm * (BM / 2) + i * 16 + lane % 16) * kLdsRow + kk +
                                         (lane / 16) * 8);
#pragma unroll
            for (int j = 0; j < TN; ++j)
                bf[j] = *(const f16x8 *)(Bs(cur) + (wn * (BN / 2) + j * 16 + lane % 16) * kLdsRow + kk +
                                         (lane / 16) * 8);
#pragma unroll
            for (int i = 0; i < TM; ++i)
#pragma unroll
                for (int j = 0; j < TN; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[i], bf[j], acc[i][j], 0, 0, 0);
        }
        if (more)
            stash(cur ^ 1);
        __syncthreads();
        cur ^= 1;
    }

    // lane holds C[4*(lane/16) + e][lane % 16] of each 16x16 block
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
#pragma unroll
            for (int e = 0; e < 4; ++e)
            {
                const uint32_t m = m0 + wm * (BM / 2) + i * 16 + 4 * (lane / 16) + e;
                const uint32_t n = n0 + wn * (BN / 2) + j * 16 + lane % 16;
                if (m >= M || n >= N)
                    continue;
                if (SPLIT)
                    work[((size_t)blockIdx.y * M + m) * N + n] = acc[i][j][e];
                else
                    gemm_store(EPI, C, ldc, m, n, acc[i][j][e], split);
            }
}

// The same product on v_mfma_f32_32x32x16_f16 with larger wave tiles: 4 waves as 2 x 2 of (BM/2) x (BN/2), each a
// grid of 32x32 MFMA blocks (up to 4 x 4: 256 fp32 accumulators per lane). A wave tile of 128 x 128 reads half the
// LDS bytes per flop of a 64 x 64 one. Operands: lane l holds row (l % 32) of a 32-row block at K offset
// 8 (l / 32) of each 16-wide K slice; the block's accumulator element e of lane l is C[8 (e / 4) + 4 (l / 32) +
// e % 4][l % 32]. Loads, LDS layout, tile order and split-K as in gemm_kernel.
typedef float f32x16 __attribute__((ext_vector_type(16)));

// f(integral_constant<int, J>) for J in the sequence, in order
template <int... J, typename F>
__device__ __forceinline__ void for_seq(std::integer_sequence<int, J...>, F &&f)
{
    (f(std::integral_constant<int, J>{}), ...);
}

// PF: K steps whose global loads are in flight at once. With PF 2 the loads run two steps ahead through two register
// sets (a step's loads are stored to LDS at the end of the following step); a split tile of a short prompt has little
// MFMA work per step, and one step of loads in flight leaves it waiting on memory latency every step. PF 4 (four
// register sets, 128 x 128 tiles only, one workgroup per CU for the registers) keeps the whole K of a short prompt's
// tile in one workgroup.
// n_base: product column of the kernel's column 0 (B rows and C columns are addressed from it; N counts the
// kernel's columns). GEMM_SWIGLU reads the product's columns from [Wu; Wg] as interleaved 32-row blocks and
// `split` holds F.
template <int BM, int BN, int EPI, bool SPLIT, int PF = 1>
__global__ __launch_bounds__(256, (PF > 2 ? 1 : PF)) void gemm32_kernel(const uint16_t *__restrict__ A,
                                                        const uint16_t *__restrict__ B, uint16_t *C, float *work,
                                                        uint32_t M, uint32_t N, uint32_t K, uint32_t ldc,
                                                        uint32_t split, uint32_t kchunk, uint32_t tiles_m,
                                                        uint32_t tiles_total, uint32_t n_base, GemmRope rope)
{
    constexpr int WM = BM / 2, WN = BN / 2, TM = WM / 32, TN = WN / 32;
    constexpr int AV = BM * kBK / 8 / 256, BV = BN * kBK / 8 / 256; // 16-byte vectors per thread per K step
    extern __shared__ __attribute__((aligned(16))) uint16_t lds[];
    auto As = [&](int b) { return lds + b * BM * kLdsRow; };
    auto Bs = [&](int b) { return lds + 2 * BM * kLdsRow + b * BN * kLdsRow; };

    const uint32_t per_xcd = gridDim.x / 8;
    const uint32_t t = (blockIdx.x % 8) * per_xcd + blockIdx.x / 8;
    if (t >= tiles_total)
        return;
    const uint32_t m0 = (t % tiles_m) * BM, n0 = (t / tiles_m) * BN;
    const uint32_t kb = SPLIT ? blockIdx.y * kchunk : 0;
    const uint32_t ke = SPLIT ? min(K, kb + kchunk) : K;
    const uint32_t tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
    const uint32_t wm = wid >> 1, wn = wid & 1;

    f32x16 acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
#pragma unroll
            for (int e = 0; e < 16; ++e)
                acc[i][j][e] = 0.f;

    // every K step lies wholly inside [kb, ke) (the launcher admits K ranges of whole 64-wide steps), so the
    // loads need no masks and each step's body is straight-line code for the scheduler
    u32x4 ra[PF][AV], rb[PF][BV];
    // element offsets of this thread's B rows (fixed for the tile) at its 16-byte column of a K step; B has fewer
    // than 2^32 elements (checked by the launcher)
    uint32_t boff[BV];
#pragma unroll
    for (int i = 0; i < BV; ++i)
    {
        const uint32_t v = tid + 256 * i;
        boff[i] = gemm_b_row<EPI>(n_base + min(n0 + v / 8, N - 1), split) * K + (v % 8) * 8;
    }
    auto load = [&](auto set_tag, uint32_t k0) {
        constexpr int S = decltype(set_tag)::value;
#pragma unroll
        for (int i = 0; i < AV; ++i)
        {
            const uint32_t v = tid + 256 * i, row = min(m0 + v / 8, M - 1);
            ra[S][i] = *(const u32x4 *)(A + (size_t)row * K + k0 + (v % 8) * 8);
        }
#pragma unroll
        for (int i = 0; i < BV; ++i)
            rb[S][i] = __builtin_nontemporal_load((const u32x4 *)(B + boff[i] + k0));
    };
    auto stash = [&](auto set_tag, int buf) {
        constexpr int S = decltype(set_tag)::value;
#pragma unroll
        for (int i = 0; i < AV; ++i)
        {
            const uint32_t v = tid + 256 * i;
            *(u32x4 *)(As(buf) + (v / 8) * kLdsRow + (v % 8) * 8) = ra[S][i];
        }
#pragma unroll
        for (int i = 0; i < BV; ++i)
        {
            const uint32_t v = tid + 256 * i;
            *(u32x4 *)(Bs(buf) + (v / 8) * kLdsRow + (v % 8) * 8) = rb[S][i];
        }
    };
    f16x8 af[2][TM], bf[2][TN];
    auto frags = [&](int buf, int slice, int into) {
#pragma unroll
        for (int i = 0; i < TM; ++i)
            af[into][i] = *(const f16x8 *)(As(buf) + (wm * WM + i * 32 + lane % 32) * kLdsRow + slice * 16 +
                                           (lane / 32) * 8);
#pragma unroll
        for (int j = 0; j < TN; ++j)
            bf[into][j] = *(const f16x8 *)(Bs(buf) + (wn * WN + j * 32 + lane % 32) * kLdsRow + slice * 16 +
                                           (lane / 32) * 8);
    };
    auto mfmas = [&](int from) {
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int j = 0; j < TN; ++j)
                acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[from][i], bf[from][j], acc[i][j], 0, 0, 0);
    };
    // One K step from LDS buffer `buf`. With LD, global loads of step `kload` go to register set LS during the first
    // slice; with ST, register set SS is stored to the other LDS buffer during the last one. The group barriers lay
    // the instruction stream out as MFMAs with the operand reads of the next slice, the global loads and the LDS
    // stores threaded between them.
    constexpr int NMF = TM * TN, NDR = TM + TN, NLD = AV + BV;
    constexpr int LD_PER = (NLD + NMF - 1) / NMF;
    auto step = [&](auto ld_tag, auto st_tag, auto ls_tag, auto ss_tag, int buf, uint32_t kload) {
        constexpr bool LD = decltype(ld_tag)::value, ST = decltype(st_tag)::value;
        frags(buf, 0, 0);
        frags(buf, 1, 1);
        if constexpr (LD)
            load(ls_tag, kload);
        mfmas(0);
        frags(buf, 2, 0);
        mfmas(1);
        frags(buf, 3, 1);
        mfmas(0);
        mfmas(1);
        if constexpr (ST)
            stash(ss_tag, buf ^ 1);
        // slice 0 operands first, then: slice 0 MFMAs with slice 1 reads and the global loads, slices 1 and 2 with
        // the next slice's reads, slice 3 with the LDS stores
        __builtin_amdgcn_sched_group_barrier(0x100, NDR, 0);
#pragma unroll
        for (int i = 0; i < NMF; ++i)
        {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
            if (i < NDR)
                __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
            if (LD && i * LD_PER < NLD)
                __builtin_amdgcn_sched_group_barrier(0x020, LD_PER, 0);
        }
#pragma unroll
        for (int sl = 1; sl < 3; ++sl)
#pragma unroll
            for (int i = 0; i < NMF; ++i)
            {
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                if (i < NDR)
                    __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
            }
#pragma unroll
        for (int i = 0; i < NMF; ++i)
        {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
            if (ST && i * LD_PER < NLD)
                __builtin_amdgcn_sched_group_barrier(0x200, LD_PER, 0);
        }
    };

    using T = std::true_type;
    using F = std::false_type;
    using S0 = std::integral_constant<int, 0>;
    using S1 = std::integral_constant<int, PF - 1>;
    const uint32_t nsteps = (ke - kb) / kBK;
    if constexpr (PF == 1)
    {
        load(S0{}, kb);
        stash(S0{}, 0);
        __syncthreads();
        int cur = 0;
        uint32_t k0 = kb;
        for (; k0 + kBK < ke; k0 += kBK)
        {
            step(T{}, T{}, S0{}, S0{}, cur, k0 + kBK);
            __syncthreads();
            cur ^= 1;
        }
        step(F{}, F{}, S0{}, S0{}, cur, k0);
    }
    else if constexpr (PF > 2)
    {
        // Step s computes from LDS buffer s % 2 while register sets hold steps s + 1 .. s + PF - 1 in flight: it
        // loads step s + PF into set s % PF (free since step s went to LDS) and stores set (s + 1) % PF into buffer
        // (s + 1) % 2. Loads past the last step re-read the last step (L2 hits), so every step is the same code and
        // the wait before each store covers only the set being stored. Steps run in groups of PF (static set
        // indices), the last nsteps % PF in a tail of straight-line steps.
        static_assert(PF % 2 == 0, "PF > 2 must be even (buffer parity follows the set index)");
        const uint32_t lastk = kb + (nsteps - 1) * kBK;
        auto kat = [&](uint32_t st) { return st < nsteps ? kb + st * kBK : lastk; };
        for_seq(std::make_integer_sequence<int, PF>{}, [&](auto j) { load(j, kat(decltype(j)::value)); });
        stash(S0{}, 0);
        __syncthreads();
        uint32_t s = 0;
        auto run_steps = [&](auto seq) {
            for_seq(seq, [&](auto j) {
                constexpr int J = decltype(j)::value;
                step(T{}, T{}, j, std::integral_constant<int, (J + 1) % PF>{}, J % 2, kat(s + J + PF));
                __syncthreads();
            });
        };
        for (; s + PF <= nsteps; s += PF)
            run_steps(std::make_integer_sequence<int, PF>{});
        const uint32_t left = nsteps - s;
        if constexpr (PF >= 4)
        {
            if (left == 3)
                run_steps(std::make_integer_sequence<int, 3>{});
            else if (left == 2)
                run_steps(std::make_integer_sequence<int, 2>{});
            else if (left == 1)
                run_steps(std::make_integer_sequence<int, 1>{});
        }
        static_assert(PF <= 4, "tail covers at most 3 steps");
    }
    else
    {
        // step s computes from LDS buffer s % 2, loads step s + 2 into register set s % 2 and stores set
        // (s + 1) % 2 (step s + 1, loaded during step s - 1) into buffer (s + 1) % 2; pairs keep the sets static
        load(S0{}, kb);
        load(S1{}, nsteps > 1 ? kb + kBK : kb); // unconditional: storing set 0 then waits for set 0 only
        stash(S0{}, 0);
        __syncthreads();
        uint32_t s = 0;
        for (; s + 3 < nsteps; s += 2)
        {
            step(T{}, T{}, S0{}, S1{}, 0, kb + (s + 2) * kBK);
            __syncthreads();
            step(T{}, T{}, S1{}, S0{}, 1, kb + (s + 3) * kBK);
            __syncthreads();
        }
        const uint32_t left = nsteps - s; // 1, 2 or 3 steps, the first from buffer 0
        if (left == 3)
        {
            step(T{}, T{}, S0{}, S1{}, 0, kb + (s + 2) * kBK);
            __syncthreads();
            step(F{}, T{}, S1{}, S0{}, 1, 0);
            __syncthreads();
            step(F{}, F{}, S0{}, S0{}, 0, 0);
        }
        else if (left == 2)
        {
            step(F{}, T{}, S0{}, S1{}, 0, 0);
            __syncthreads();
            step(F{}, F{}, S1{}, S1{}, 1, 0);
        }
        else
            step(F{}, F{}, S0{}, S0{}, 0, 0);
    }

    if constexpr (!SPLIT)
    {
        // Epilogue through LDS (the K-step buffers are free now): each lane writes its fp16 outputs into a row-major
        // tile, then the workgroup moves 16-byte row chunks to their destinations, so the stores (and the residual's
        // loads) are whole vectors instead of one 2-byte element per lane. SwiGLU tiles have BN / 2 output columns.
        constexpr int OC = EPI == GEMM_SWIGLU ? BN / 2 : BN;
        constexpr int TROW = OC + 8; // halves; rows 4 apart then start 16 banks apart
        static_assert(BM * TROW <= 2 * (BM + BN) * kLdsRow, "epilogue tile fits the K-step buffers");
        __syncthreads();
        uint16_t *T = lds;
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int j = 0; j < TN; j += (EPI == GEMM_SWIGLU ? 2 : 1))
#pragma unroll
                for (int e = 0; e < 16; ++e)
                {
                    const uint32_t rt = wm * WM + i * 32 + 8 * (e / 4) + 4 * (lane / 32) + e % 4;
                    const uint32_t ct = wn * WN + j * 32 + lane % 32;
                    if constexpr (EPI == GEMM_SWIGLU)
                        T[rt * TROW + swiglu_col(ct)] = swiglu_out(acc[i][j][e], acc[i][j + 1][e]);
                    else if constexpr (EPI == GEMM_SILU_HI)
                        T[rt * TROW + ct] = f2h(n_base + n0 + ct >= split ? silu(acc[i][j][e]) : acc[i][j][e]);
                    else
                        T[rt * TROW + ct] = f2h(acc[i][j][e]);
                }
        __syncthreads();
        constexpr int CH = OC / 8;
        const uint32_t oc0 = EPI == GEMM_SWIGLU ? (n_base + n0) / 2 : n_base + n0; // output column of tile column 0
        const uint32_t oce = EPI == GEMM_SWIGLU ? (n_base + N) / 2 : n_base + N;   // end of this launch's columns
        const bool vec = ((uintptr_t)C % 16 == 0) && ldc % 8 == 0;
        for (uint32_t idx = tid; idx < (uint32_t)(BM * CH); idx += 256)
        {
            const uint32_t rt = idx / CH, m = m0 + rt, col = oc0 + (idx % CH) * 8;
            if (m >= M || col >= oce)
                continue;
            const uint16_t *t = T + rt * TROW + (idx % CH) * 8;
            if constexpr (EPI == GEMM_QKV_ROPE)
                rope_store8(rope, m, col, *(const u32x4 *)t); // N is a multiple of 64: whole chunks
            else
            {
                uint16_t *c = C + (size_t)m * ldc + col;
                const uint32_t cnt = min(8u, oce - col);
                if (vec && cnt == 8)
                {
                    u32x4 v = *(const u32x4 *)t;
                    if constexpr (EPI == GEMM_RESID)
                    {
                        const u32x4 r = *(const u32x4 *)c;
#pragma unroll
                        for (int k = 0; k < 4; ++k)
                            v[k] = pack2(f2h(h2f((uint16_t)r[k]) + half_lo(v[k])),
                                         f2h(h2f((uint16_t)(r[k] >> 16)) + half_hi(v[k])));
                    }
                    *(u32x4 *)c = v;
                }
                else
                    for (uint32_t k = 0; k < cnt; ++k)
                        c[k] = EPI == GEMM_RESID ? f2h(h2f(c[k]) + h2f(t[k])) : t[k];
            }
        }
        return;
    }
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
#pragma unroll
            for (int e = 0; e < 16; ++e)
            {
                const uint32_t m = m0 + wm * WM + i * 32 + 8 * (e / 4) + 4 * (lane / 32) + e % 4;
                const uint32_t n = n0 + wn * WN + j * 32 + lane % 32;
                if (m < M && n < N)
                    work[((size_t)blockIdx.y * M + m) * N + n] = acc[i][j][e];
            }
}

// C = epilogue(sum over z of work[z]) for split-K products, the splits added in order
// whether the plain, SiLU and residual epilogues of the split-K reduce can move 8 columns as one 16-byte vector
__host__ __device__ __forceinline__ bool reduce_vec8(uint32_t N, uint32_t ldc, uint32_t n_base, const uint16_t *C)
{
    return N % 8 == 0 && ldc % 8 == 0 && n_base % 8 == 0 && (uintptr_t)C % 16 == 0;
}

template <int EPI>
__global__ __launch_bounds__(256) void gemm_splitk_reduce_kernel(const float *work, uint16_t *C, uint32_t M,
                                                                 uint32_t N, uint32_t ldc, uint32_t split,
                                                                 uint32_t splits, uint32_t n_base, GemmRope rope)
{
    const uint64_t total = (uint64_t)M * N;
    // 8 consecutive columns per step (N % 64 == 0 for these epilogues): 16-byte partial loads and output stores
    auto sum8 = [&](size_t at, float *v) {
#pragma unroll
        for (int k = 0; k < 8; ++k)
            v[k] = 0.f;
        for (uint32_t z = 0; z < splits; ++z)
        {
            const float4 *p = (const float4 *)(work + (size_t)z * total + at);
            const float4 a = p[0], b = p[1];
            v[0] += a.x;
            v[1] += a.y;
            v[2] += a.z;
            v[3] += a.w;
            v[4] += b.x;
            v[5] += b.y;
            v[6] += b.z;
            v[7] += b.w;
        }
    };
    if constexpr (EPI == GEMM_QKV_ROPE)
    {
        const uint32_t per_row = N / 8;
        const uint64_t chunks = (uint64_t)M * per_row;
        for (uint64_t i = (uint64_t)blockIdx.x * 256 + threadIdx.x; i < chunks; i += (uint64_t)gridDim.x * 256)
        {
            const uint32_t m = (uint32_t)(i / per_row), n = 8 * (uint32_t)(i % per_row);
            float v[8];
            sum8((size_t)m * N + n, v);
            u32x4 h;
#pragma unroll
            for (int k = 0; k < 4; ++k)
                h[k] = pack2(f2h(v[2 * k]), f2h(v[2 * k + 1]));
            rope_store8(rope, m, n_base + n, h);
        }
        return;
    }
    if constexpr (EPI == GEMM_SWIGLU)
    {
        // 8 output columns f..f + 7 (inside one 32-column block): up columns c..c + 7, gate columns c + 32..c + 39
        const uint32_t per_row = N / 16;
        const uint64_t chunks = (uint64_t)M * per_row;
        for (uint64_t i = (uint64_t)blockIdx.x * 256 + threadIdx.x; i < chunks; i += (uint64_t)gridDim.x * 256)
        {
            const uint32_t m = (uint32_t)(i / per_row), f = 8 * (uint32_t)(i % per_row), c = 64 * (f / 32) + f % 32;
            float up[8], gate[8];
            sum8((size_t)m * N + c, up);
            sum8((size_t)m * N + c + 32, gate);
            u32x4 o;
#pragma unroll
            for (int k = 0; k < 4; ++k)
                o[k] = pack2(swiglu_out(up[2 * k], gate[2 * k]), swiglu_out(up[2 * k + 1], gate[2 * k + 1]));
            *(u32x4 *)(C + (size_t)m * ldc + swiglu_col(n_base + c)) = o;
        }
        return;
    }
    if (reduce_vec8(N, ldc, n_base, C))
    {
        // 8 consecutive columns per step: 16-byte partial loads and one 16-byte store (the same sums, in the same
        // split order, as the element loop below)
        const uint32_t per_row = N / 8;
        const uint64_t chunks = (uint64_t)M * per_row;
        for (uint64_t i = (uint64_t)blockIdx.x * 256 + threadIdx.x; i < chunks; i += (uint64_t)gridDim.x * 256)
        {
            const uint32_t m = (uint32_t)(i / per_row), n = 8 * (uint32_t)(i % per_row);
            float v[8];
            sum8((size_t)m * N + n, v);
            uint16_t *c = C + (size_t)m * ldc + n_base + n;
            u32x4 o;
            if constexpr (EPI == GEMM_RESID)
            {
                const u32x4 old = *(const u32x4 *)c;
#pragma unroll
                for (int k = 0; k < 4; ++k)
                    o[k] = pack2(f2h(half_lo(old[k]) + h2f(f2h(v[2 * k]))),
                                 f2h(half_hi(old[k]) + h2f(f2h(v[2 * k + 1]))));
            }
            else
            {
#pragma unroll
                for (int k = 0; k < 8; ++k)
                    if (EPI == GEMM_SILU_HI && n_base + n + k >= split)
                        v[k] = silu(v[k]);
#pragma unroll
                for (int k = 0; k < 4; ++k)
                    o[k] = pack2(f2h(v[2 * k]), f2h(v[2 * k + 1]));
            }
            *(u32x4 *)c = o;
        }
        return;
    }
    for (uint64_t i = (uint64_t)blockIdx.x * 256 + threadIdx.x; i < total; i += (uint64_t)gridDim.x * 256)
    {
        float v = 0.f;
        for (uint32_t z = 0; z < splits; ++z)
            v += work[(size_t)z * total + i];
        gemm_store(EPI, C, ldc, (uint32_t)(i / N), n_base + (uint32_t)(i % N), v, split);
    }
}

// work items of gemm_splitk_reduce_kernel: 8 columns each where the epilogue or reduce_vec8 allows, else one element
template <int EPI>
static uint32_t reduce_grid(uint32_t M, uint32_t N, uint32_t ldc, uint32_t n_base, const uint16_t *C)
{
    uint64_t items = (uint64_t)M * N;
    if (EPI == GEMM_SWIGLU)
        items /= 16;
    else if (EPI == GEMM_QKV_ROPE || reduce_vec8(N, ldc, n_base, C))
        items /= 8;
    const uint64_t grid = (items + 255) / 256;
    return (uint32_t)(grid > 4096 ? 4096 : grid < 1 ? 1 : grid);
}

// Split-K residual products followed by RMSNorm (every residual product of the token step is): one workgroup per
// row m, C[m] = fp16(C[m] + fp16(sum over z of work[z][m])) with the splits added in order (as the reduce kernel),
// then y[m] = RMSNorm(C[m]) * w as rmsnorm_row_to computes it, with launch_rmsnorm_rows's block size (so the same
// sum order). Each thread re-reads only the vectors it wrote.
__global__ __launch_bounds__(512) void gemm_resid_norm_kernel(const float *work, uint16_t *C, uint32_t M, uint32_t N,
                                                              uint32_t splits, const float *w, uint16_t *y,
                                                              float eps, bool xt)
{
    __shared__ float red[8];
    const uint32_t m = blockIdx.x, nv = N / 8;
    const size_t total = (size_t)M * N;
    u32x4 *cv = (u32x4 *)(C + (size_t)m * N);
    for (uint32_t i = threadIdx.x; i < nv; i += blockDim.x)
    {
        float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll 8
        for (uint32_t z = 0; z < splits; ++z)
        {
            const float4 *p = (const float4 *)(work + z * total + (size_t)m * N + 8 * i);
            const float4 a = p[0], b = p[1];
            acc[0] += a.x;
            acc[1] += a.y;
            acc[2] += a.z;
            acc[3] += a.w;
            acc[4] += b.x;
            acc[5] += b.y;
            acc[6] += b.z;
            acc[7] += b.w;
        }
        const u32x4 r = cv[i];
        u32x4 o;
#pragma unroll
        for (int k = 0; k < 4; ++k)
            o[k] = pack2(f2h(half_lo(r[k]) + h2f(f2h(acc[2 * k]))), f2h(half_hi(r[k]) + h2f(f2h(acc[2 * k + 1]))));
        cv[i] = o;
    }
    if (xt)
        rmsnorm_row_to(C + (size_t)m * N, w, (u32x4 *)y, N, eps, red, (int)m);
    else
        rmsnorm_row_to(C + (size_t)m * N, w, (u32x4 *)(y + (size_t)m * N), N, eps, red);
}

// gemm_resid_norm_kernel for rows of at most 512 VPT vectors: each thread keeps its vectors in registers from the
// partial sums to the normalised output, and requests the residual and norm weights with the partials, so the row
// makes one round trip to memory instead of three. The sums run in the same order (a thread's vectors ascending,
// the same block_sum), so the outputs equal the generic kernel's bit for bit.
template <int VPT>
__global__ __launch_bounds__(512) void gemm_resid_norm_regs_kernel(const float *work, uint16_t *C, uint32_t M,
                                                                   uint32_t N, uint32_t splits, const float *w,
                                                                   uint16_t *y, float eps, bool xt)
{
    __shared__ float red[8];
    const uint32_t m = blockIdx.x, nv = N / 8, tid = threadIdx.x;
    const size_t total = (size_t)M * N;
    u32x4 *cv = (u32x4 *)(C + (size_t)m * N);
    const float4 *wv = (const float4 *)w;
    // unconditional loads at clamped indices (a guarded load compiles to a branch and a wait per load)
    u32x4 r[VPT];
    float4 wa[VPT], wb[VPT];
#pragma unroll
    for (int j = 0; j < VPT; ++j)
    {
        const uint32_t i = min(tid + 512 * j, nv - 1);
        r[j] = cv[i];
        wa[j] = wv[2 * i];
        wb[j] = wv[2 * i + 1];
    }
    float ss = 0.f;
#pragma unroll
    for (int j = 0; j < VPT; ++j)
    {
        const uint32_t i = tid + 512 * j;
        const uint32_t ic = min(i, nv - 1);
        float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll 8
        for (uint32_t z = 0; z < splits; ++z)
        {
            const float4 *p = (const float4 *)(work + z * total + (size_t)m * N + 8 * ic);
            const float4 a = p[0], b = p[1];
            acc[0] += a.x;
            acc[1] += a.y;
            acc[2] += a.z;
            acc[3] += a.w;
            acc[4] += b.x;
            acc[5] += b.y;
            acc[6] += b.z;
            acc[7] += b.w;
        }
#pragma unroll
        for (int k = 0; k < 4; ++k)
            r[j][k] = pack2(f2h(half_lo(r[j][k]) + h2f(f2h(acc[2 * k]))),
                            f2h(half_hi(r[j][k]) + h2f(f2h(acc[2 * k + 1]))));
        if (i < nv)
        {
            cv[i] = r[j];
#pragma unroll
            for (int k = 0; k < 4; ++k)
            {
                const float a = half_lo(r[j][k]), b = half_hi(r[j][k]);
                ss += a * a;
                ss += b * b;
            }
        }
    }
    ss = block_sum(ss, red);
    const float alpha = 1.0f / sqrtf(ss / (float)N + eps);
#pragma unroll
    for (int j = 0; j < VPT; ++j)
    {
        const uint32_t i = tid + 512 * j;
        if (i >= nv)
            continue;
        const float ws[8] = {wa[j].x, wa[j].y, wa[j].z, wa[j].w, wb[j].x, wb[j].y, wb[j].z, wb[j].w};
        u32x4 o;
#pragma unroll
        for (int k = 0; k < 4; ++k)
        {
            const float a = half_lo(r[j][k]), b = half_hi(r[j][k]);
            o[k] = pack2(f2h((a * ws[2 * k]) * alpha), f2h((b * ws[2 * k + 1]) * alpha));
        }
        ((u32x4 *)y)[xt ? xt_vec(m, i) : (size_t)m * nv + i] = o;
    }
}

// the residual-norm reduce for a row of N columns (one 512-thread workgroup per row)
static hipError_t launch_resid_norm(hipStream_t st, const float *work, uint16_t *C, uint32_t M, uint32_t N,
                                    uint32_t splits, const GemmNorm &norm)
{
    const uint32_t nv = N / 8;
    if (nv <= 512)
        gemm_resid_norm_regs_kernel<1><<<M, 512, 0, st>>>(work, C, M, N, splits, norm.w, norm.y, norm.eps, norm.xt);
    else if (nv <= 1024)
        gemm_resid_norm_regs_kernel<2><<<M, 512, 0, st>>>(work, C, M, N, splits, norm.w, norm.y, norm.eps, norm.xt);
    else
        gemm_resid_norm_kernel<<<M, 512, 0, st>>>(work, C, M, N, splits, norm.w, norm.y, norm.eps, norm.xt);
    return hipGetLastError();
}

template <int BM, int BN> static size_t gemm_lds()
{
    return (size_t)2 * (BM + BN) * kLdsRow * sizeof(uint16_t);
}

template <int BM, int BN, int EPI, bool SPLIT>
static hipError_t launch_tile(hipStream_t st, const uint16_t *A, const uint16_t *B, uint16_t *C, float *work,
                              uint32_t M, uint32_t N, uint32_t K, uint32_t ldc, uint32_t split, uint32_t splits,
                              uint32_t kchunk)
{
    static uint64_t attr_devs = 0; // devices on which the LDS limit is raised for this kernel
    const size_t lds = gemm_lds<BM, BN>();
    hipError_t e = lds_attr_once((const void *)gemm_kernel<BM, BN, EPI, SPLIT>, lds, attr_devs);
    if (e != hipSuccess)
        return e;
    const uint32_t tm = (M + BM - 1) / BM, tn = (N + BN - 1) / BN, total = tm * tn;
    const uint32_t grid = (total + 7) / 8 * 8;
    gemm_kernel<BM, BN, EPI, SPLIT><<<dim3(grid, SPLIT ? splits : 1), 256, lds, st>>>(A, B, C, work, M, N, K, ldc,
                                                                                     split, kchunk, tm, total);
    return hipGetLastError();
}

template <int BM, int BN, int EPI, bool SPLIT, int PF = 1>
static hipError_t launch_tile32(hipStream_t st, const uint16_t *A, const uint16_t *B, uint16_t *C, float *work,
                                uint32_t M, uint32_t N, uint32_t K, uint32_t ldc, uint32_t split, uint32_t splits,
                                uint32_t kchunk, uint32_t n_base = 0, const GemmRope *rope = nullptr)
{
    static uint64_t attr_devs = 0; // devices on which the LDS limit is raised for this kernel
    const size_t lds = gemm_lds<BM, BN>();
    hipError_t e = lds_attr_once((const void *)gemm32_kernel<BM, BN, EPI, SPLIT, PF>, lds, attr_devs);
    if (e != hipSuccess)
        return e;
    const uint32_t tm = (M + BM - 1) / BM, tn = (N + BN - 1) / BN, total = tm * tn;
    const uint32_t grid = (total + 7) / 8 * 8;
    gemm32_kernel<BM, BN, EPI, SPLIT, PF><<<dim3(grid, SPLIT ? splits : 1), 256, lds, st>>>(
        A, B, C, work, M, N, K, ldc, split, kchunk, tm, total, n_base, rope ? *rope : GemmRope{});
    return hipGetLastError();
}

template <int EPI>
static hipError_t launch_reduce(hipStream_t st, const float *work, uint16_t *C, uint32_t M, uint32_t N, uint32_t ldc,
                                uint32_t split, uint32_t splits, uint32_t n_base, const GemmRope *rope)
{
    const uint32_t grid = reduce_grid<EPI>(M, N, ldc, n_base, C);
    gemm_splitk_reduce_kernel<EPI>
        <<<grid, 256, 0, st>>>(work, C, M, N, ldc, split, splits, n_base, rope ? *rope : GemmRope{});
    return hipGetLastError();
}

template <int BM, int BN, int EPI>
static hipError_t launch_shape32(hipStream_t st, const uint16_t *A, const uint16_t *B, uint16_t *C, float *work,
                                 uint32_t M, uint32_t N, uint32_t K, uint32_t ldc, uint32_t split, uint32_t splits,
                                 uint32_t kchunk, uint32_t n_base = 0, const GemmRope *rope = nullptr)
{
    if (splits <= 1)
        return launch_tile32<BM, BN, EPI, false>(st, A, B, C, work, M, N, K, ldc, split, 1, K, n_base, rope);
    // split tiles (short prompts): two K steps of loads in flight where the registers allow it
    constexpr int PF = BM * BN <= 128 * 128 ? 2 : 1;
    hipError_t e = launch_tile32<BM, BN, EPI, true, PF>(st, A, B, C, work, M, N, K, ldc, split, splits, kchunk,
                                                        n_base, rope);
    if (e != hipSuccess)
        return e;
    return launch_reduce<EPI>(st, work, C, M, N, ldc, split, splits, n_base, rope);
}

template <int BM, int BN, int EPI>
static hipError_t launch_shape(hipStream_t st, const uint16_t *A, const uint16_t *B, uint16_t *C, float *work,
                               uint32_t M, uint32_t N, uint32_t K, uint32_t ldc, uint32_t split, uint32_t splits,
                               uint32_t kchunk)
{
    if (splits <= 1)
        return launch_tile<BM, BN, EPI, false>(st, A, B, C, work, M, N, K, ldc, split, 1, K);
    hipError_t e = launch_tile<BM, BN, EPI, true>(st, A, B, C, work, M, N, K, ldc, split, splits, kchunk);
    if (e != hipSuccess)
        return e;
    const uint32_t grid = reduce_grid<EPI>(M, N, ldc, 0, C);
    gemm_splitk_reduce_kernel<EPI><<<grid, 256, 0, st>>>(work, C, M, N, ldc, split, splits, 0, GemmRope{});
    return hipGetLastError();
}

template <int EPI>
static hipError_t launch_epi_gemm(hipStream_t st, const uint16_t *A, const uint16_t *B, uint16_t *C, float *work,
                                  size_t work_elems, uint32_t M, uint32_t N, uint32_t K, uint32_t ldc,
                                  uint32_t split, int cu_count, const GemmRope *rope, const GemmNorm *norm,
                                  bool *normed)
{
    const uint32_t cus = cu_count > 0 ? (uint32_t)cu_count : 256;
    if constexpr (EPI == GEMM_QKV_ROPE)
        if (!rope || K % kBK != 0 || rope->D % 64 != 0 || rope->hd < 32 || (rope->hd & (rope->hd - 1)) != 0 ||
            N != 3 * rope->D || !rope->cs)
            return hipErrorInvalidValue;
    if ((uint64_t)N * K >= (1ull << 32)) // B row offsets are 32-bit
        return hipErrorInvalidValue;
    if constexpr (EPI == GEMM_SWIGLU)
        if (K % kBK != 0 || N % 64 != 0 || N != 2 * split || ldc % 8 != 0 || (uintptr_t)C % 16 != 0)
            return hipErrorInvalidValue;
    if (K % kBK == 0)
    {
        // 32x32x16 kernel: 256 x 256 tiles when they alone give most CUs a tile; else 128 x 128 tiles (two fit a
        // CU) with K split until about two workgroups per CU run, or 1.4 for prompts of at most 128 tokens (their
        // partial tiles cost more than further splits gain), each split keeping at least 256 of K
        const uint64_t t256 = (uint64_t)((M + 255) / 256) * ((N + 255) / 256);
        // also when 128 x 128 tiles would take more rounds: a pair of them on a CU takes about 2/3 of a 256 x 256
        // tile's time (13B Wo and down at 2048 tokens: 160 tiles, 141 and 395 us against 189 and 514 us)
        const uint64_t r256 = (t256 + cus - 1) / cus, r128 = (2 * t256 + cus - 1) / cus;
        if (t256 >= (cus * 3) / 4 || r128 * 2 > r256 * 3)
        {
            // Residual products whose 256 x 256 tiles make one partial round: 128 x 320 tiles when they give at
            // least 1.5 times as many CUs a tile in one round (13B Wo and down at 2048 tokens: 256 tiles for 256
            // CUs instead of 160; Wo + Wd 528 -> 485 us per layer, outputs bit-identical, since every output adds its
            // K terms in the same order in either tile). The same tiles were slower for the plain vocabulary product,
            // and 128 x 384 tiles level for the 7B QKV product at 1024 tokens.
            if constexpr (EPI == GEMM_RESID)
            {
                const uint64_t t320 = (uint64_t)((M + 127) / 128) * ((N + 319) / 320);
                if (t256 < cus && t320 <= cus && t320 * 2 >= t256 * 3)
                    return launch_tile32<128, 320, EPI, false, 1>(st, A, B, C, work, M, N, K, ldc, split, 1, K);
            }
            // A last round of 256 x 256 tiles at most half full would leave most CUs idle for a whole tile's time:
            // its tile columns run as a product of their own with K split over those CUs (partials added in order
            // by the reduce), the full rounds as before.
            const uint32_t tm = (M + 255) / 256, tn = (N + 255) / 256;
            const uint64_t full = t256 / cus, rem = t256 % cus;
            if (full >= 1 && rem > 0 && rem * 2 <= cus)
            {
                const uint32_t tail_cols = (uint32_t)((rem + tm - 1) / tm), n_split = (tn - tail_cols) * 256;
                const uint32_t tail_n = N - n_split;
                uint32_t splits = cus / (tm * tail_cols);
                while (splits > 1 && (K / splits < 4 * kBK || (size_t)splits * M * tail_n > work_elems))
                    --splits;
                if (splits >= 2)
                {
                    const uint32_t kchunk = ((K + splits - 1) / splits + kBK - 1) / kBK * kBK;
                    hipError_t e =
                        launch_shape32<256, 256, EPI>(st, A, B, C, work, M, n_split, K, ldc, split, 1, K, 0, rope);
                    if (e != hipSuccess)
                        return e;
                    return launch_shape32<256, 256, EPI>(st, A, B, C, work, M, tail_n, K, ldc, split,
                                                         (K + kchunk - 1) / kchunk, kchunk, n_split, rope);
                }
            }
            return launch_shape32<256, 256, EPI>(st, A, B, C, work, M, N, K, ldc, split, 1, K, 0, rope);
        }
        // Residual products of long rows (K >= 5120: 13B Wo, 7B and 13B down) above 128 tokens whose 256 x 256 tiles
        // leave most CUs idle: K split s ways so that one round of 256 x 256 tiles fills at least three quarters of
        // the CUs, each split keeping at least 1280 of K. Against the 128 x 128 path: 7B down at 1024 tokens 110 vs
        // 135 us (4 splits), 13B down 145 vs 250 us (3), 13B Wo 84 vs 108 us (3), 7B down at 640 tokens 92 vs 127 us
        // (5), 7 to 30% at 384-2048 tokens; 7B Wo (K 4096) is level or slower at every length and stays on 128 x 128.
        if constexpr (EPI == GEMM_RESID)
        {
            const uint32_t s = t256 > 0 ? (uint32_t)(cus / t256) : 0;
            if (M > 128 && K >= 5120 && s >= 2 && t256 * s * 4 >= (uint64_t)cus * 3 && K / s >= 1280 &&
                (size_t)s * M * N <= work_elems)
            {
                const uint32_t kchunk = ((K + s - 1) / s + kBK - 1) / kBK * kBK, ns = (K + kchunk - 1) / kchunk;
                hipError_t e =
                    launch_tile32<256, 256, EPI, true, 1>(st, A, B, C, work, M, N, K, ldc, split, ns, kchunk);
                if (e != hipSuccess)
                    return e;
                if (norm)
                {
                    *normed = true;
                    return launch_resid_norm(st, work, C, M, N, ns, *norm);
                }
                return launch_reduce<EPI>(st, work, C, M, N, ldc, split, ns, 0, nullptr);
            }
        }
        const uint64_t tiles = (uint64_t)((M + 127) / 128) * ((N + 127) / 128);
        // prompts of at most 128 tokens whose tiles cover two thirds of the CUs or more ([Wu;Wg], logits): the
        // whole K per tile with four K steps of loads in flight (one workgroup per CU) beats split K and its reduce
        if (M <= 128 && tiles * 3 >= (uint64_t)cus * 2)
            return launch_tile32<128, 128, EPI, false, 4>(st, A, B, C, work, M, N, K, ldc, split, 1, K, 0, rope);
        // workgroups per CU, times 10. Plain products above 128 tokens (the MATMUL op's) split K only until one
        // workgroup per CU runs: a second workgroup per CU leaves the tile kernel no faster and doubles the partials
        // the reduce reads (M 512, N = K = 4096: 128 tiles x 2 K ranges 29.7 + 5.4 us, x 4 ranges 30.2 + 8.2 us)
        const uint64_t per_cu10 = M <= 128 ? 14 : EPI == GEMM_PLAIN ? 10 : 20;
        uint32_t splits = 1;
        while (tiles * splits * 2 * 10 <= per_cu10 * cus && K / (splits * 2) >= 256 &&
               (size_t)splits * 2 * M * N <= work_elems)
            splits *= 2;
        const uint32_t kchunk = ((K + splits - 1) / splits + kBK - 1) / kBK * kBK;
        splits = (K + kchunk - 1) / kchunk;
        if constexpr (EPI == GEMM_RESID)
            if (norm && splits > 1)
            {
                // the reduce adds the residual and normalises the updated rows in one pass
                hipError_t e = launch_tile32<128, 128, EPI, true, 2>(st, A, B, C, work, M, N, K, ldc, split, splits,
                                                                     kchunk);
                if (e != hipSuccess)
                    return e;
                // 512 threads a row (one 16-byte vector each at width 4096) keep a row's partial loads in flight
                *normed = true;
                return launch_resid_norm(st, work, C, M, N, splits, *norm);
            }
        return launch_shape32<128, 128, EPI>(st, A, B, C, work, M, N, K, ldc, split, splits, kchunk, 0, rope);
    }
    if constexpr (EPI == GEMM_SWIGLU || EPI == GEMM_QKV_ROPE)
        return hipErrorInvalidValue; // checked above: not reached
    else
    {
        if (M <= 128)
        {
            // weight-streaming regime: a 128-row tile covers all of M so each weight is read once; K is split over
            // workgroups when N is narrow
            const uint32_t tiles = (N + 63) / 64;
            uint32_t splits = 1;
            while (tiles * splits <= cus && K / (splits * 2) >= 512 && (size_t)splits * 2 * M * N <= work_elems)
                splits *= 2;
            const uint32_t kchunk = ((K + splits - 1) / splits + kBK - 1) / kBK * kBK;
            splits = (K + kchunk - 1) / kchunk;
            return launch_shape<128, 64, EPI>(st, A, B, C, work, M, N, K, ldc, split, splits, kchunk);
        }
        const uint64_t big = (uint64_t)((M + 127) / 128) * ((N + 127) / 128);
        if (big >= cus)
            return launch_shape<128, 128, EPI>(st, A, B, C, work, M, N, K, ldc, split, 1, K);
        return launch_shape<128, 64, EPI>(st, A, B, C, work, M, N, K, ldc, split, 1, K);
    }
}

hipError_t launch_gemm_reduce(hipStream_t st, int epi, const float *work, uint16_t *C, uint32_t M, uint32_t N,
                              uint32_t splits, const GemmRope *rope, const GemmNorm *norm)
{
    if (M == 0 || N == 0 || splits == 0)
        return hipErrorInvalidValue;
    switch (epi)
    {
    case GEMM_RESID:
        if (!norm)
            return launch_reduce<GEMM_RESID>(st, work, C, M, N, N, 0, splits, 0, nullptr);
        if (N % 8 != 0 || (norm->xt && (M > 128 || N % 16 != 0)))
            return hipErrorInvalidValue;
        return launch_resid_norm(st, work, C, M, N, splits, *norm);
    case GEMM_QKV_ROPE:
        if (!rope || N != 3 * rope->D)
            return hipErrorInvalidValue;
        return launch_reduce<GEMM_QKV_ROPE>(st, work, C, M, N, N, 0, splits, 0, rope);
    default:
        return hipErrorInvalidValue;
    }
}

hipError_t launch_gemm(hipStream_t st, int epi, const uint16_t *A, const uint16_t *B, uint16_t *C, uint32_t M,
                       uint32_t N, uint32_t K, uint32_t ldc, uint32_t split, int cu_count, float *work,
                       size_t work_elems, const GemmRope *rope, const GemmNorm *norm)
{
    if (K % 8 != 0 || K < 8 || M == 0 || N == 0)
        return hipErrorInvalidValue;
    switch (epi)
    {
    case GEMM_PLAIN:
        return launch_epi_gemm<GEMM_PLAIN>(st, A, B, C, work, work_elems, M, N, K, ldc, split, cu_count, nullptr,
                                             nullptr, nullptr);
    case GEMM_SILU_HI:
        return launch_epi_gemm<GEMM_SILU_HI>(st, A, B, C, work, work_elems, M, N, K, ldc, split, cu_count, nullptr,
                                             nullptr, nullptr);
    case GEMM_RESID:
    {
        if (norm && (ldc != N || N % 8 != 0))
            return hipErrorInvalidValue;
        bool normed = false;
        hipError_t e = launch_epi_gemm<GEMM_RESID>(st, A, B, C, work, work_elems, M, N, K, ldc, split, cu_count,
                                                   nullptr, norm, &normed);
        if (e != hipSuccess || !norm || normed)
            return e;
        return launch_rmsnorm_rows(st, C, norm->w, norm->y, M, N, norm->eps, norm->xt);
    }
    case GEMM_SWIGLU:
        return launch_epi_gemm<GEMM_SWIGLU>(st, A, B, C, work, work_elems, M, N, K, ldc, split, cu_count, nullptr,
                                             nullptr, nullptr);
    case GEMM_QKV_ROPE:
        return launch_epi_gemm<GEMM_QKV_ROPE>(st, A, B, C, work, work_elems, M, N, K, ldc, split, cu_count, rope,
                                              nullptr, nullptr);
    default:
        return hipErrorInvalidValue;
    }
}

} // namespace vk
