// Stride-aware gfx950 kernels behind the VKLLM_OP_* operators (node-by-node execution and the op API).
// They implement the operator semantics of the reference's shaders (src/shaders/*.comp) for any dtype mix and
// any element strides; the LLaMA-2 token step itself runs on the fused kernels (fused_*.hip).
#include <float.h>

#include "device_common.h"
#include "kernels.h"

namespace vk
{

static inline uint32_t blocks_for(uint64_t n, uint32_t bs)
{
    return (uint32_t)((n + bs - 1) / bs);
}

static inline uint64_t numel(const TView &t)
{
    return (uint64_t)t.n[0] * t.n[1] * t.n[2] * t.n[3];
}

// ---------------------------------------------------------------------------------------------------------------
// VKLLM_OP_COPY (src/shaders/vkllm_copy.comp:35-50) and VKLLM_OP_UPDATE_ROWS
// (src/shaders/vkllm_update_rows.comp:21-46): raw element moves, bit-exact.
template <typename T>
__global__ void copy_kernel(TView in, TView out, uint64_t total, uint32_t row_offset)
{
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += (uint64_t)gridDim.x * blockDim.x)
    {
        uint32_t b, c, h, w;
        unflatten(i, in.n, b, c, h, w);
        if (h + row_offset >= out.n[2])
            continue;
        ((T *)out.p)[voff(out, b, c, h + row_offset, w)] = ((const T *)in.p)[voff(in, b, c, h, w)];
    }
}

static hipError_t launch_move(hipStream_t st, const TView &in, const TView &out, uint32_t row_offset)
{
    uint64_t total = numel(in);
    if (total == 0)
        return hipSuccess;
    uint32_t grid = blocks_for(total, 256);
    grid = grid > 65536 ? 65536 : grid;
    switch (in.dt)
    {
    case DT_F16:
        copy_kernel<uint16_t><<<grid, 256, 0, st>>>(in, out, total, row_offset);
        break;
    case DT_I8:
        copy_kernel<uint8_t><<<grid, 256, 0, st>>>(in, out, total, row_offset);
        break;
    default:
        copy_kernel<uint32_t><<<grid, 256, 0, st>>>(in, out, total, row_offset);
        break;
    }
    return hipGetLastError();
}

hipError_t launch_copy(hipStream_t st, const TView &in, const TView &out)
{
    return launch_move(st, in, out, 0);
}

hipError_t launch_update_rows(hipStream_t st, const TView &src, const TView &cache, uint32_t offset_rows)
{
    return launch_move(st, src, cache, offset_rows);
}

// ---------------------------------------------------------------------------------------------------------------
// VKLLM_OP_BIN (src/shaders/vkllm_bin_op.comp:41-73): fp32 arithmetic, result rounded to the output dtype.
__global__ void bin_kernel(TView a, TView b, TView out, int op, uint64_t total)
{
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += (uint64_t)gridDim.x * blockDim.x)
    {
        uint32_t n, c, h, w;
        unflatten(i, out.n, n, c, h, w);
        float x = ldf(a, voff(a, n, c, h, w)), y = ldf(b, voff(b, n, c, h, w));
        float r = op == 0 ? x + y : op == 1 ? x - y : op == 2 ? x * y : x / y;
        stf(out, voff(out, n, c, h, w), r);
    }
}

hipError_t launch_bin(hipStream_t st, const TView &a, const TView &b, const TView &out, int op)
{
    uint64_t total = numel(out);
    uint32_t grid = blocks_for(total, 256);
    grid = grid > 65536 ? 65536 : grid;
    bin_kernel<<<grid, 256, 0, st>>>(a, b, out, op, total);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------------------------------------------
// VKLLM_OP_EMBEDDING (src/shaders/vkllm_embedding.comp:41-70): one workgroup per index; index (0, c, h, w)
// writes output row c*s0 + h*s1 + w*s2; ids >= rows read row `unk`.
__global__ void embedding_kernel(TView idx, TView table, TView out, uint32_t unk)
{
    uint32_t b, c, h, w;
    unflatten(blockIdx.x, idx.n, b, c, h, w);
    uint32_t tok = ((const uint32_t *)idx.p)[voff(idx, b, c, h, w)];
    const uint32_t rows = table.n[2], D = table.n[3];
    if (tok >= rows)
        tok = unk;
    if (tok >= rows)
        return;
    size_t o = (size_t)c * out.s[0] + (size_t)h * out.s[1] + (size_t)w * out.s[2];
    size_t p = (size_t)tok * table.s[2];
    if (table.dt == DT_F16)
        for (uint32_t i = threadIdx.x; i < D; i += blockDim.x)
            ((uint16_t *)out.p)[o + (size_t)i * out.s[3]] = ((const uint16_t *)table.p)[p + (size_t)i * table.s[3]];
    else
        for (uint32_t i = threadIdx.x; i < D; i += blockDim.x)
            ((uint32_t *)out.p)[o + (size_t)i * out.s[3]] = ((const uint32_t *)table.p)[p + (size_t)i * table.s[3]];
}

hipError_t launch_embedding(hipStream_t st, const TView &idx, const TView &table, const TView &out, uint32_t unk)
{
    uint64_t n = numel(idx);
    if (n == 0)
        return hipSuccess;
    embedding_kernel<<<(uint32_t)n, 256, 0, st>>>(idx, table, out, unk);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------------------------------------------
// VKLLM_OP_RMSNORM (src/shaders/vkllm_rmsnorm.comp:31-82): alpha = 1/sqrt(sum(x^2)/W + eps), y = (x*w)*alpha.
__global__ void rmsnorm_kernel(TView x, TView wt, TView out, float eps)
{
    __shared__ float red[16];
    uint32_t b, c, h, w;
    const uint32_t n3[4] = {x.n[0], x.n[1], x.n[2], 1};
    unflatten(blockIdx.x, n3, b, c, h, w);
    const uint32_t W = x.n[3];
    size_t xr = voff(x, b, c, h, 0), orow = voff(out, b, c, h, 0);
    float ss = 0.f;
    for (uint32_t i = threadIdx.x; i < W; i += blockDim.x)
    {
        float v = ldf(x, xr + (size_t)i * x.s[3]);
        ss += v * v;
    }
    ss = block_sum(ss, red);
    float mean = ss / (float)W;
    float alpha = 1.0f / sqrtf(mean + eps);
    for (uint32_t i = threadIdx.x; i < W; i += blockDim.x)
    {
        float v0 = ldf(x, xr + (size_t)i * x.s[3]);
        float v1 = ldf(wt, (size_t)i * wt.s[3]);
        stf(out, orow + (size_t)i * out.s[3], (v0 * v1) * alpha);
    }
}

hipError_t launch_rmsnorm(hipStream_t st, const TView &x, const TView &w, const TView &out, float eps)
{
    uint64_t rows = (uint64_t)x.n[0] * x.n[1] * x.n[2];
    if (rows == 0)
        return hipSuccess;
    rmsnorm_kernel<<<(uint32_t)rows, 256, 0, st>>>(x, w, out, eps);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------------------------------------------
// VKLLM_OP_MATMUL and VKLLM_OP_FFN_UP_AND_GATE, generic path: 64x64 output tile per 256-thread workgroup, 4x4 per
// thread, K staged through LDS in steps of 16, fp32 accumulation. Operands of any dtype and strides; size-1
// batch/channel dims broadcast (src/core/vkllm_op_matmul.c:32-63). With DUAL, a second B operand gives
// out = acc0 * silu(acc1) (src/shaders/vkllm_ffn_up_and_gate.comp:133-147).
constexpr int GT = 64, GK = 16;

template <bool DUAL>
__global__ __launch_bounds__(256) void gemm_generic_kernel(TView a, TView b0, TView b1, TView out, float scale,
                                                           int act, int transposed_b)
{
    __shared__ float As[GK][GT + 1];
    __shared__ float Bs[DUAL ? 2 : 1][GK][GT + 1];
    const uint32_t M = out.n[2], N = out.n[3], K = a.n[3];
    const uint32_t bz = blockIdx.z / out.n[1], cz = blockIdx.z % out.n[1];
    const uint32_t m0 = blockIdx.x * GT, n0 = blockIdx.y * GT;
    const uint32_t ab = a.n[0] == 1 ? 0 : bz, ac = a.n[1] == 1 ? 0 : cz;
    const uint32_t bb = b0.n[0] == 1 ? 0 : bz, bc = b0.n[1] == 1 ? 0 : cz;
    const int tx = threadIdx.x % 16, ty = threadIdx.x / 16;
    float acc[2][4][4] = {};
    for (uint32_t k0 = 0; k0 < K; k0 += GK)
    {
        for (int e = threadIdx.x; e < GT * GK; e += 256)
        {
            int r = e / GK, kk = e % GK;
            uint32_t m = m0 + r, k = k0 + kk;
            As[kk][r] = (m < M && k < K) ? ldf(a, voff(a, ab, ac, m, k)) : 0.f;
            uint32_t n = n0 + r;
            bool ok = n < N && k < K;
#pragma unroll
            for (int q = 0; q < (DUAL ? 2 : 1); ++q)
            {
                const TView &bv = q == 0 ? b0 : b1;
                Bs[q][kk][r] = ok ? (transposed_b ? ldf(bv, voff(bv, bb, bc, n, k)) : ldf(bv, voff(bv, bb, bc, k, n)))
                                  : 0.f;
            }
        }
        __syncthreads();
#pragma unroll
        for (int kk = 0; kk < GK; ++kk)
        {
            float av[4], bv[2][4];
#pragma unroll
            for (int i = 0; i < 4; ++i)
                av[i] = As[kk][ty * 4 + i];
#pragma unroll
            for (int q = 0; q < (DUAL ? 2 : 1); ++q)
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    bv[q][j] = Bs[q][kk][tx * 4 + j];
#pragma unroll
            for (int q = 0; q < (DUAL ? 2 : 1); ++q)
#pragma unroll
                for (int i = 0; i < 4; ++i)
#pragma unroll
                    for (int j = 0; j < 4; ++j)
                        acc[q][i][j] = fmaf(av[i], bv[q][j], acc[q][i][j]);
        }
        __syncthreads();
    }
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j)
        {
            uint32_t m = m0 + ty * 4 + i, n = n0 + tx * 4 + j;
            if (m >= M || n >= N)
                continue;
            float v;
            if (DUAL)
            {
                float g = acc[1][i][j];
                v = acc[0][i][j] * g / (1.0f + expf(-g));
            }
            else
            {
                v = acc[0][i][j] * scale;
                if (act == 1)
                    v = silu(v);
            }
            stf(out, voff(out, bz, cz, m, n), v);
        }
}

// M == 1 with B [N, K] (the reference's mat_mul_vec case, src/shaders/vkllm_mat_mul_vec.comp:94-150): one wave per
// output element, lanes striding K.
__global__ __launch_bounds__(256) void gemv_generic_kernel(TView a, TView b, TView out, float scale, int act)
{
    const uint32_t N = out.n[3];
    const uint64_t total = (uint64_t)out.n[0] * out.n[1] * N;
    const uint64_t wid = (uint64_t)blockIdx.x * (blockDim.x / kWave) + threadIdx.x / kWave;
    const int lane = threadIdx.x % kWave;
    if (wid >= total)
        return;
    const uint32_t n = (uint32_t)(wid % N), cz = (uint32_t)((wid / N) % out.n[1]), bz = (uint32_t)(wid / N / out.n[1]);
    const uint32_t ab = a.n[0] == 1 ? 0 : bz, ac = a.n[1] == 1 ? 0 : cz;
    const uint32_t bb = b.n[0] == 1 ? 0 : bz, bc = b.n[1] == 1 ? 0 : cz;
    const uint32_t K = a.n[3];
    float acc = 0.f;
    for (uint32_t k = lane; k < K; k += kWave)
        acc = fmaf(ldf(a, voff(a, ab, ac, 0, k)), ldf(b, voff(b, bb, bc, n, k)), acc);
    acc = wave_sum(acc);
    if (lane == 0)
    {
        float v = acc * scale;
        if (act == 1)
            v = silu(v);
        stf(out, voff(out, bz, cz, 0, n), v);
    }
}

hipError_t launch_matmul(hipStream_t st, const TView &a, const TView &b, const TView &out, float scale, int act,
                         bool transposed_b)
{
    const uint32_t M = out.n[2], N = out.n[3];
    const uint64_t batches = (uint64_t)out.n[0] * out.n[1];
    if (M == 0 || N == 0 || batches == 0)
        return hipSuccess;
    if (M == 1 && transposed_b)
    {
        uint64_t waves = batches * N;
        gemv_generic_kernel<<<blocks_for(waves, 4), 256, 0, st>>>(a, b, out, scale, act);
        return hipGetLastError();
    }
    dim3 grid(blocks_for(M, GT), blocks_for(N, GT), (uint32_t)batches);
    gemm_generic_kernel<false><<<grid, 256, 0, st>>>(a, b, b, out, scale, act, transposed_b ? 1 : 0);
    return hipGetLastError();
}

hipError_t launch_ffn_up_and_gate(hipStream_t st, const TView &x, const TView &wu, const TView &wg, const TView &out)
{
    const uint32_t M = out.n[2], N = out.n[3];
    const uint64_t batches = (uint64_t)out.n[0] * out.n[1];
    if (M == 0 || N == 0 || batches == 0)
        return hipSuccess;
    dim3 grid(blocks_for(M, GT), blocks_for(N, GT), (uint32_t)batches);
    gemm_generic_kernel<true><<<grid, 256, 0, st>>>(x, wu, wg, out, 1.0f, 0, 1);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------------------------------------------
// VKLLM_OP_ROPE (src/shaders/vkllm_rope.comp:39-79): one thread per rotated pair.
struct RopeFreqs
{
    float f[kMaxRopeFreqs];
};

__global__ void rope_kernel(TView in, TView out, uint32_t offset, RopeFreqs fr, int neox, uint64_t total)
{
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += (uint64_t)gridDim.x * blockDim.x)
    {
        const uint32_t half = in.n[3] / 2;
        const uint32_t n4[4] = {in.n[0], in.n[1], in.n[2], half};
        uint32_t b, c, h, w;
        unflatten(i, n4, b, c, h, w);
        size_t i0, i1, o0, o1;
        if (neox)
        {
            i0 = voff(in, b, c, h, w);
            i1 = i0 + (size_t)in.s[3] * half;
            o0 = voff(out, b, c, h, w);
            o1 = o0 + (size_t)out.s[3] * half;
        }
        else
        {
            i0 = voff(in, b, c, h, 2 * w);
            i1 = i0 + in.s[3];
            o0 = voff(out, b, c, h, 2 * w);
            o1 = o0 + out.s[3];
        }
        float f = (float)(offset + h) / fr.f[w];
        float fc = cosf(f), fs = sinf(f);
        float v0 = ldf(in, i0), v1 = ldf(in, i1);
        stf(out, o0, fc * v0 - fs * v1);
        stf(out, o1, fs * v0 + fc * v1);
    }
}

// fp16 views whose rows (the W axis) are contiguous and 16-byte aligned, the layout of both the isolated operator and
// the model's permuted Q/K views: one workgroup per (position h, batch b) computes the row's cos/sin pairs once into
// LDS, then rotates 16-byte vectors of every channel with them. Each pair's angle and its cosf/sinf are those of
// rope_kernel, and so are the products, so the outputs are identical.
__global__ __launch_bounds__(256) void rope_rows_kernel(TView in, TView out, uint32_t offset, RopeFreqs fr, int neox)
{
    __shared__ float cs[2 * kMaxRopeFreqs];
    const uint32_t h = blockIdx.x, b = blockIdx.y;
    const uint32_t half = in.n[3] / 2, C = in.n[1];
    const uint16_t *src = (const uint16_t *)in.p;
    uint16_t *dst = (uint16_t *)out.p;
    // vectors of the row per channel: 4 adjacent pairs (2w, 2w + 1) each, or with neox 8 pairs (w, w + half) as a
    // vector of the low half and the matching one of the high half
    const uint32_t nv = neox ? half / 8 : in.n[3] / 8, items = C * nv;
    auto at_lo = [&](const TView &t, uint32_t i) { return voff(t, b, i / nv, h, 8 * (i % nv)); };
    auto at_hi = [&](const TView &t, uint32_t i) { return voff(t, b, i / nv, h, half + 8 * (i % nv)); };
    // the first kPre items of every thread are requested before the angle table is computed, so their memory
    // latency overlaps the cosf / sinf work (the isolated [1, 32, 512, 128] operator: all of a workgroup's items)
    constexpr int kPre = 2;
    u32x4 plo[kPre], phi[kPre];
#pragma unroll
    for (int p = 0; p < kPre; ++p)
    {
        const uint32_t i = threadIdx.x + p * blockDim.x;
        if (i < items)
        {
            plo[p] = *(const u32x4 *)(src + at_lo(in, i));
            phi[p] = neox ? *(const u32x4 *)(src + at_hi(in, i)) : plo[p];
        }
    }
    for (uint32_t w = threadIdx.x; w < half; w += blockDim.x)
    {
        const float f = (float)(offset + h) / fr.f[w];
        cs[2 * w] = cosf(f);
        cs[2 * w + 1] = sinf(f);
    }
    __syncthreads();
    auto rotate = [&](uint32_t i, const u32x4 &lo, const u32x4 &hi) {
        const uint32_t v = i % nv;
        if (!neox)
        {
            u32x4 o;
#pragma unroll
            for (int k = 0; k < 4; ++k)
            {
                const uint32_t w = 4 * v + k;
                const float fc = cs[2 * w], fs = cs[2 * w + 1];
                const float v0 = half_lo(lo[k]), v1 = half_hi(lo[k]);
                o[k] = pack2(f2h(fc * v0 - fs * v1), f2h(fs * v0 + fc * v1));
            }
            *(u32x4 *)(dst + at_lo(out, i)) = o;
            return;
        }
        u32x4 olo, ohi;
#pragma unroll
        for (int k = 0; k < 4; ++k)
        {
            const uint32_t w0 = 8 * v + 2 * k, w1 = w0 + 1;
            const float a0 = half_lo(lo[k]), b0 = half_lo(hi[k]), a1 = half_hi(lo[k]), b1 = half_hi(hi[k]);
            olo[k] = pack2(f2h(cs[2 * w0] * a0 - cs[2 * w0 + 1] * b0), f2h(cs[2 * w1] * a1 - cs[2 * w1 + 1] * b1));
            ohi[k] = pack2(f2h(cs[2 * w0 + 1] * a0 + cs[2 * w0] * b0), f2h(cs[2 * w1 + 1] * a1 + cs[2 * w1] * b1));
        }
        *(u32x4 *)(dst + at_lo(out, i)) = olo;
        *(u32x4 *)(dst + at_hi(out, i)) = ohi;
    };
#pragma unroll
    for (int p = 0; p < kPre; ++p)
    {
        const uint32_t i = threadIdx.x + p * blockDim.x;
        if (i < items)
            rotate(i, plo[p], phi[p]);
    }
    for (uint32_t i = threadIdx.x + kPre * blockDim.x; i < items; i += blockDim.x)
    {
        const u32x4 lo = *(const u32x4 *)(src + at_lo(in, i));
        const u32x4 hi = neox ? *(const u32x4 *)(src + at_hi(in, i)) : lo;
        rotate(i, lo, hi);
    }
}

static bool rope_rows_ok(const TView &t, bool neox)
{
    const uint32_t W = t.n[3];
    return t.dt == DT_F16 && t.s[3] == 1 && (neox ? (W / 2) % 8 == 0 : W % 8 == 0) && t.s[2] % 8 == 0 &&
           t.s[1] % 8 == 0 && t.s[0] % 8 == 0 && (uintptr_t)t.p % 16 == 0 && t.n[0] <= 65535;
}

hipError_t launch_rope(hipStream_t st, const TView &in, const TView &out, uint32_t offset, const float *freqs_host,
                       bool neox)
{
    RopeFreqs fr;
    const uint32_t half = in.n[3] / 2;
    if (half > (uint32_t)kMaxRopeFreqs)
        return hipErrorInvalidValue;
    for (uint32_t w = 0; w < half; ++w)
        fr.f[w] = freqs_host[w];
    uint64_t total = (uint64_t)in.n[0] * in.n[1] * in.n[2] * half;
    if (total == 0)
        return hipSuccess;
    if (rope_rows_ok(in, neox) && rope_rows_ok(out, neox))
    {
        rope_rows_kernel<<<dim3(in.n[2], in.n[0]), 256, 0, st>>>(in, out, offset, fr, neox ? 1 : 0);
        return hipGetLastError();
    }
    uint32_t grid = blocks_for(total, 256);
    grid = grid > 65536 ? 65536 : grid;
    rope_kernel<<<grid, 256, 0, st>>>(in, out, offset, fr, neox ? 1 : 0, total);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------------------------------------------
// VKLLM_OP_SOFTMAX (src/shaders/vkllm_softmax.comp:42-96): max over the whole row; with seq_mask, entries
// i > h + offsets are excluded from the sum and written as 0.
__global__ void softmax_kernel(TView in, TView out, int seq_mask, uint32_t offsets)
{
    __shared__ float red[16];
    uint32_t b, c, h, w;
    const uint32_t n3[4] = {out.n[0], out.n[1], out.n[2], 1};
    unflatten(blockIdx.x, n3, b, c, h, w);
    const uint32_t W = out.n[3];
    size_t ir = voff(in, b, c, h, 0), orow = voff(out, b, c, h, 0);
    float mx = -FLT_MAX;
    for (uint32_t i = threadIdx.x; i < W; i += blockDim.x)
        mx = fmaxf(mx, ldf(in, ir + (size_t)i * in.s[3]));
    mx = block_max(mx, red);
    const uint32_t lim = h + offsets;
    float sum = 0.f;
    for (uint32_t i = threadIdx.x; i < W; i += blockDim.x)
        if (!(seq_mask > 0 && i > lim))
            sum += expf(ldf(in, ir + (size_t)i * in.s[3]) - mx);
    sum = block_sum(sum, red);
    for (uint32_t i = threadIdx.x; i < W; i += blockDim.x)
    {
        float v = (seq_mask > 0 && i > lim) ? 0.f : expf(ldf(in, ir + (size_t)i * in.s[3]) - mx) / sum;
        stf(out, orow + (size_t)i * out.s[3], v);
    }
}

hipError_t launch_softmax(hipStream_t st, const TView &in, const TView &out, int seq_mask, uint32_t offsets)
{
    uint64_t rows = (uint64_t)out.n[0] * out.n[1] * out.n[2];
    if (rows == 0)
        return hipSuccess;
    softmax_kernel<<<(uint32_t)rows, 256, 0, st>>>(in, out, seq_mask, offsets);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------------------------------------------
// VKLLM_OP_ARG_MAX (src/shaders/vkllm_arg_max.comp:40-97) on any strided view: each thread keeps the first element
// of its share under the reference's arg-max order (am_before), then wave shuffles and one LDS step reduce the
// row. Contiguous fp16 rows take the fused step's 16-byte-load kernel (launch_argmax_rows).
__global__ __launch_bounds__(256) void arg_max_kernel(TView in, TView out)
{
    __shared__ float wv[4];
    __shared__ uint32_t wi[4];
    uint32_t b, c, h, w;
    const uint32_t n3[4] = {in.n[0], in.n[1], in.n[2], 1};
    unflatten(blockIdx.x, n3, b, c, h, w);
    const uint32_t W = in.n[3];
    const size_t row = voff(in, b, c, h, 0);
    const uint32_t t = threadIdx.x;
    float bv = -INFINITY;
    uint32_t bi = 0xFFFFFFFFu; // no element: every element comes before it
    if (t >= W && t < 32)
    {
        // the reference's lanes past a row shorter than 32 enter its reduction with (-FLT_MAX, lane)
        // (src/shaders/vkllm_arg_max.comp:55-60): elements of their own here, ahead of a row of -inf
        bv = -FLT_MAX;
        bi = t;
    }
    for (uint32_t i = t; i < W; i += 256)
    {
        const float v = ldf(in, row + (size_t)i * in.s[3]);
        if (am_before(v, i, bv, bi))
        {
            bv = v;
            bi = i;
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
        for (int k = 1; k < 4; ++k)
            if (am_before(wv[k], wi[k], bv, bi))
            {
                bv = wv[k];
                bi = wi[k];
            }
        ((uint32_t *)out.p)[voff(out, b, c, h, 0)] = bi;
    }
}

static bool contiguous(const TView &t)
{
    return t.s[3] == 1 && t.s[2] == t.n[3] && t.s[1] == t.n[2] * t.s[2] && t.s[0] == t.n[1] * t.s[1];
}

hipError_t launch_arg_max(hipStream_t st, const TView &in, const TView &out)
{
    uint64_t rows = (uint64_t)in.n[0] * in.n[1] * in.n[2];
    if (rows == 0)
        return hipSuccess;
    if (in.dt == DT_F16 && contiguous(in) && contiguous(out))
        return launch_argmax_rows(st, (const uint16_t *)in.p, (uint32_t *)out.p, (uint32_t)rows, in.n[3]);
    arg_max_kernel<<<(uint32_t)rows, 256, 0, st>>>(in, out);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------------------------------------------
// synthetic weights
__device__ __forceinline__ uint64_t splitmix64(uint64_t stream, uint64_t n)
{
    uint64_t z = stream + (n + 1) * 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

__global__ void random_f16_kernel(uint16_t *dst, uint64_t count, uint64_t key, float std)
{
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < count; i += (uint64_t)gridDim.x * blockDim.x)
    {
        int32_t sum = 0;
#pragma unroll
        for (int r = 0; r < 3; ++r)
        {
            uint64_t v = splitmix64(key, 3 * i + (uint64_t)r);
#pragma unroll
            for (int k = 0; k < 4; ++k)
                sum += (int32_t)((v >> (16 * k)) & 0xffffu);
        }
        float z = (float)(sum + 6 - 6 * 65536) / 65536.0f;
        dst[i] = f2h(z * std);
    }
}

hipError_t launch_random_f16(hipStream_t st, uint16_t *dst, uint64_t count, uint64_t stream_key, float std)
{
    if (count == 0)
        return hipSuccess;
    uint32_t grid = blocks_for(count, 256);
    grid = grid > 8192 ? 8192 : grid;
    random_f16_kernel<<<grid, 256, 0, st>>>(dst, count, stream_key, std);
    return hipGetLastError();
}

__global__ void fill_f32_kernel(float *dst, uint64_t count, float v)
{
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < count; i += (uint64_t)gridDim.x * blockDim.x)
        dst[i] = v;
}

hipError_t launch_fill_f32(hipStream_t st, float *dst, uint64_t count, float v)
{
    if (count == 0)
        return hipSuccess;
    uint32_t grid = blocks_for(count, 256);
    grid = grid > 8192 ? 8192 : grid;
    fill_f32_kernel<<<grid, 256, 0, st>>>(dst, count, v);
    return hipGetLastError();
}

} // namespace vk
