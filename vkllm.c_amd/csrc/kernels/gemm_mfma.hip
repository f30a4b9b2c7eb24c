// Prefill GEMM on CDNA4 matrix cores: C[M, N] = A[M, K] . B[N, K]^T with fp16 operands and fp32 accumulation
// (v_mfma_f32_16x16x32_f16), the dense replacement for src/shaders/vkllm_matmul_t1.comp on the token step's
// weight products.
//
// Tiling: BM x BN output tile per 256-thread workgroup (2 x 2 waves, each (BM/2) x (BN/2) as 16x16 MFMA blocks),
// K in steps of 32. Tiles of A and B go through LDS with rows padded to 80 bytes, which keeps the 16-lane
// ds_read_b128 operand fetches on distinct banks; the next K step's global loads are issued before the current
// step's MFMAs. Tiles are ordered M-fastest and dealt to XCDs in contiguous runs so a run shares its B tiles in
// one L2.
#include "device_common.h"
#include "kernels.h"

namespace vk
{

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4g __attribute__((ext_vector_type(4)));

constexpr int kBK = 32;
constexpr int kLdsRow = kBK + 8; // halfs per LDS row (80 bytes)

template <int BM, int BN, int EPI>
__global__ __launch_bounds__(256) void gemm_kernel(const uint16_t *__restrict__ A, const uint16_t *__restrict__ B,
                                                   uint16_t *C, uint32_t M, uint32_t N, uint32_t K, uint32_t ldc,
                                                   uint32_t split, uint32_t tiles_m, uint32_t tiles_total)
{
    constexpr int TM = BM / 32, TN = BN / 32; // 16x16 blocks per wave
    constexpr int AV = BM * 4 / 256, BV = BN * 4 / 256; // 16-byte vectors per thread per K step
    __shared__ __attribute__((aligned(16))) uint16_t As[BM * kLdsRow];
    __shared__ __attribute__((aligned(16))) uint16_t Bs[BN * kLdsRow];

    const uint32_t per_xcd = gridDim.x / 8;
    const uint32_t t = (blockIdx.x % 8) * per_xcd + blockIdx.x / 8;
    if (t >= tiles_total)
        return;
    const uint32_t m0 = (t % tiles_m) * BM, n0 = (t / tiles_m) * BN;
    const uint32_t tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
    const uint32_t wm = wid >> 1, wn = wid & 1;

    f32x4 acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
            acc[i][j] = (f32x4){0.f, 0.f, 0.f, 0.f};

    u32x4g ra[AV], rb[BV];
    // unconditional loads at clamped addresses (a guarded load compiles to a branch and a wait per load): rows
    // past M or N only feed outputs that are not stored; K columns past the end are zeroed by a select
    auto load = [&](uint32_t k0) {
#pragma unroll
        for (int i = 0; i < AV; ++i)
        {
            const uint32_t v = tid + 256 * i, row = min(m0 + v / 4, M - 1), kk = k0 + (v % 4) * 8;
            const u32x4g x = *(const u32x4g *)(A + (size_t)row * K + min(kk, K - 8));
            ra[i] = kk < K ? x : (u32x4g){0, 0, 0, 0};
        }
#pragma unroll
        for (int i = 0; i < BV; ++i)
        {
            const uint32_t v = tid + 256 * i, row = min(n0 + v / 4, N - 1), kk = k0 + (v % 4) * 8;
            const u32x4g x = *(const u32x4g *)(B + (size_t)row * K + min(kk, K - 8));
            rb[i] = kk < K ? x : (u32x4g){0, 0, 0, 0};
        }
    };

    load(0);
    for (uint32_t k0 = 0; k0 < K; k0 += kBK)
    {
#pragma unroll
        for (int i = 0; i < AV; ++i)
        {
            const uint32_t v = tid + 256 * i;
            *(u32x4g *)(As + (v / 4) * kLdsRow + (v % 4) * 8) = ra[i];
        }
#pragma unroll
        for (int i = 0; i < BV; ++i)
        {
            const uint32_t v = tid + 256 * i;
            *(u32x4g *)(Bs + (v / 4) * kLdsRow + (v % 4) * 8) = rb[i];
        }
        __syncthreads();
        if (k0 + kBK < K)
            load(k0 + kBK);
        f16x8 af[TM], bf[TN];
#pragma unroll
        for (int i = 0; i < TM; ++i)
            af[i] = *(const f16x8 *)(As + (wm * (BM / 2) + i * 16 + lane % 16) * kLdsRow + (lane / 16) * 8);
#pragma unroll
        for (int j = 0; j < TN; ++j)
            bf[j] = *(const f16x8 *)(Bs + (wn * (BN / 2) + j * 16 + lane % 16) * kLdsRow + (lane / 16) * 8);
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int j = 0; j < TN; ++j)
                acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[i], bf[j], acc[i][j], 0, 0, 0);
        __syncthreads();
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
                const float v = acc[i][j][e];
                uint16_t *c = C + (size_t)m * ldc + n;
                if (EPI == GEMM_PLAIN)
                    *c = f2h(v);
                else if (EPI == GEMM_SILU_HI)
                    *c = f2h(n >= split ? silu(v) : v);
                else
                    *c = f2h(h2f(*c) + h2f(f2h(v)));
            }
}

template <int BM, int BN>
static hipError_t launch_tile(hipStream_t st, int epi, const uint16_t *A, const uint16_t *B, uint16_t *C, uint32_t M,
                              uint32_t N, uint32_t K, uint32_t ldc, uint32_t split)
{
    const uint32_t tm = (M + BM - 1) / BM, tn = (N + BN - 1) / BN, total = tm * tn;
    const uint32_t grid = (total + 7) / 8 * 8;
    switch (epi)
    {
    case GEMM_PLAIN:
        gemm_kernel<BM, BN, GEMM_PLAIN><<<grid, 256, 0, st>>>(A, B, C, M, N, K, ldc, split, tm, total);
        break;
    case GEMM_SILU_HI:
        gemm_kernel<BM, BN, GEMM_SILU_HI><<<grid, 256, 0, st>>>(A, B, C, M, N, K, ldc, split, tm, total);
        break;
    case GEMM_RESID:
        gemm_kernel<BM, BN, GEMM_RESID><<<grid, 256, 0, st>>>(A, B, C, M, N, K, ldc, split, tm, total);
        break;
    default:
        return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_gemm(hipStream_t st, int epi, const uint16_t *A, const uint16_t *B, uint16_t *C, uint32_t M,
                       uint32_t N, uint32_t K, uint32_t ldc, uint32_t split, int cu_count)
{
    if (K % 8 != 0 || M == 0 || N == 0)
        return hipErrorInvalidValue;
    const uint64_t big_tiles = (uint64_t)((M + 127) / 128) * ((N + 127) / 128);
    if (big_tiles >= (uint64_t)(cu_count > 0 ? cu_count : 256))
        return launch_tile<128, 128>(st, epi, A, B, C, M, N, K, ldc, split);
    return launch_tile<64, 64>(st, epi, A, B, C, M, N, K, ldc, split);
}

} // namespace vk
