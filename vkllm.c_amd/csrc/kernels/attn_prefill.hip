// Prefill attention on CDNA4 matrix cores: the S query rows of a step against the kv = offset + S cached positions
// of each head (src/models/vkllm_llama2_layers.c:223-257 with src/shaders/vkllm_softmax.comp:42-96), keeping the
// reference's rounding points: s_j = fp16(scale * q.k_j); M = max over the WHOLE row (j < kv, later positions
// included, as the softmax shader takes it); L = sum of exp(s_j - M) over j <= the row's position;
// p_j = fp16(exp(s_j - M) / L) there and 0 past it; out = fp16(sum_j p_j v_j). When kv == hd the reference reads the
// V slice as [N, K] and the product becomes out[n] = fp16(sum_k p_k V[n][k]) (src/core/vkllm_op_matmul.c:14-24).
//
// A workgroup of 4 waves takes 64 query rows of one head; wave w owns rows [16 w, 16 w + 16), so every row's
// statistics stay inside one wave. Key blocks of 64 positions go through two LDS buffers (K as [key][dim], V as
// [dim][key]), shared by the 4 waves, with each block's global loads requested two blocks ahead (the kernel is
// bound by that latency, not by the matrix pipe). Products use v_mfma_f32_16x16x32_f16 in the transposed orientation:
//   S^T = K . Q^T   (A = a 16-key slice of the K tile, B = the wave's Q rows held in registers)
//   O^T += V^T . P^T (A = the V tile read as [dim][key], B = the probabilities straight from the S^T
//                     accumulators: the 32 keys of a K slice are ordered so that lane l's 8 slots are the 4 keys
//                     of each of two 16-key score blocks that it holds)
// Pass 1 walks all kv positions for M and L (an online sum, rescaled when the row max grows); pass 2 recomputes
// the same scores (same instructions, same order, so the same fp16 values) for the blocks at or before the last
// row's position and accumulates P.V. Pass 2's first two V blocks are requested at entry and its first two K blocks
// in pass 1's last step (or, for kv <= 128, read from where pass 1 left them in LDS), so pass 2 starts without a
// round trip to memory. The exponentials are the hardware's (v_exp_f32 on s log2 e - M log2 e) and p
// multiplies by 1 / L (the reference's shader leaves exp and the division to the implementation's precision as
// well). The per-score softmax arithmetic costs more issue cycles than the matrix products, so a block wholly in a
// wave's future only joins the max, and a block wholly in its past skips the masks.
#include <float.h>

#include <type_traits>

#include "device_common.h"
#include "kernels.h"

namespace vk
{

// exp(s - m) as 2^(s log2 e - m log2 e): one fused multiply-add and the hardware exponential (v_exp_f32)
constexpr float kLog2e = 1.4426950408889634f;
__device__ __forceinline__ float pf_exp2(float x)
{
    return __builtin_amdgcn_exp2f(x);
}

typedef _Float16 f16x8a __attribute__((ext_vector_type(8)));
typedef float f32x4a __attribute__((ext_vector_type(4)));

constexpr uint32_t kPfRows = 64; // query rows per workgroup
constexpr uint32_t kPfKeys = 64; // positions per key block

// K tile row pitch in halves. The score MFMA's A operand reads 16 rows x four 16-byte chunks per instruction; of the
// pitches measured on gfx950 (LDS bank-conflict counter, that read pattern alone) only 72 dwords reads without
// conflicts at head size 128; 68 and 76-132 take two passes.
template <int HD> constexpr int pf_krow()
{
    return HD == 128 ? 144 : HD + 8;
}

// max / sum over the 4 lanes that hold one row (lanes l, l ^ 16, l ^ 32, l ^ 48)
__device__ __forceinline__ float row4_max(float v)
{
    v = fmaxf(v, __shfl_xor(v, 16));
    return fmaxf(v, __shfl_xor(v, 32));
}
__device__ __forceinline__ float row4_sum(float v)
{
    v += __shfl_xor(v, 16);
    return v + __shfl_xor(v, 32);
}

// ONE: kv <= 2 key blocks, computed in one pass (below); otherwise the two passes
template <int HD, bool ONE>
__global__ __launch_bounds__(256) void attn_prefill_mfma_kernel(const uint16_t *q, const uint16_t *kc,
                                                                const uint16_t *vc, uint16_t *out, uint32_t offset,
                                                                uint32_t S, uint32_t H, uint32_t ctx, float scale,
                                                                bool xt)
{
    constexpr int KS = HD / 32;           // 32-wide slices of the head dims (K of S^T = K . Q^T)
    constexpr int DB = HD / 16;           // 16-wide blocks of output dims
    constexpr int KROW = pf_krow<HD>();   // K tile row, halves (padded for the operand reads)
    constexpr int VROW = kPfKeys + 8;     // V tile row ([dim][key]), halves (8-byte units swizzled, below)
    constexpr int KV = kPfKeys * HD / 8 / 256; // 16-byte K vectors per thread per block
    constexpr int VP = 32 * (HD / 8) / 256;    // (key pair, dim chunk) items per thread per block
    constexpr int VT = HD * (kPfKeys / 8) / 256; // transposed rule: (row, key chunk) vectors per thread
    constexpr int VR = 2 * VP > VT ? 2 * VP : VT; // V registers per set (either layout: 2 VP == VT here)
    // two buffers each of the K tile ([key][dim]) and the V tile ([dim][key]); K buffers first
    extern __shared__ __attribute__((aligned(16))) uint16_t pf_lds[];
    auto Kt = [&](int b) { return pf_lds + b * (kPfKeys * KROW); };
    auto Vt = [&](int b) { return pf_lds + 2 * kPfKeys * KROW + b * (HD * VROW); };
    // The V tile is read as 8-byte units (4 keys) by 16 lanes of 16 consecutive rows, and rows 8 apart fall on the
    // same banks (72-half rows); unit u of row r sits at u ^ ((r >> 3) & 1), so those 16 reads cover the 32 banks
    // once. Every access below has a lane-constant swizzle bit, folded into a per-lane column offset.

    const uint32_t D = H * HD, h = blockIdx.x;
    const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, q4 = lane >> 4, c16 = lane & 15;
    // heads vary fastest and row blocks run last to first: the workgroups with the most causal work start first, and
    // a head's workgroups are dealt to one XCD (blocks go to the 8 XCDs round robin) when H is a multiple of 8
    const uint32_t row0 = (gridDim.y - 1 - blockIdx.y) * kPfRows;
    const uint32_t rowc = min(row0 + wave * 16 + c16, S - 1); // this lane's query row (rows past S: not stored)
    const uint32_t pos = offset + rowc;
    const uint32_t kv = offset + S;
    const bool transposed = kv == HD;
    const uint16_t *Kh = kc + (size_t)h * ctx * HD, *Vh = vc + (size_t)h * ctx * HD;
    using S0 = std::integral_constant<int, 0>;
    using S1 = std::integral_constant<int, 1>;

    // Q^T operand: column = this lane's row, K slot 8 q4 + i = dim 32 ks + 8 q4 + i
    f16x8a qf[KS];
#pragma unroll
    for (int ks = 0; ks < KS; ++ks)
        qf[ks] = *(const f16x8a *)(q + (size_t)rowc * D + (size_t)h * HD + ks * 32 + 8 * q4);

    // V blocks 0 and 1 of pass 2, requested now: they depend on nothing, and pass 2 then starts without a round trip
    // to memory. Non-transposed, set entries [0, VP) hold keys 2 p and [VP, 2 VP) keys 2 p + 1 of the block (dims
    // [8 ch, 8 ch + 8)); transposed, entry i holds V row n, dims [jb + 8 c, jb + 8 c + 8) (the tile is read as [n][k]).
    u32x4 vr[2][VR];
    auto load_v = [&](auto set_tag, uint32_t jb) {
        constexpr int SI = decltype(set_tag)::value;
        if (!transposed)
        {
#pragma unroll
            for (int i = 0; i < VP; ++i)
            {
                const uint32_t v = tid + 256 * i, p = v % 32, ch = v / 32;
                vr[SI][i] = *(const u32x4 *)(Vh + (size_t)min(jb + 2 * p, kv - 1) * HD + ch * 8);
                vr[SI][VP + i] = *(const u32x4 *)(Vh + (size_t)min(jb + 2 * p + 1, kv - 1) * HD + ch * 8);
            }
        }
        else
        {
#pragma unroll
            for (int i = 0; i < VT; ++i)
            {
                const uint32_t v = tid + 256 * i, n = v / (kPfKeys / 8), c = v % (kPfKeys / 8);
                vr[SI][i] = *(const u32x4 *)(Vh + (size_t)n * HD + min(jb + 8 * c, (uint32_t)HD - 8));
            }
        }
    };
    load_v(S0{}, 0);
    load_v(S1{}, kPfKeys);

    // Blocks stream through two register sets and the two LDS buffers: while block b is computed from buffer
    // b % 2, set b % 2 loads block b + 2 and set (b + 1) % 2 (block b + 1, requested a block earlier) is stored to
    // the other buffer, so global loads run two blocks ahead with one barrier per block. Rows are clamped to kv - 1
    // (positions past kv are masked, whatever they hold).
    u32x4 kr[2][KV];
    auto load_k = [&](auto set_tag, uint32_t jb) {
        constexpr int SI = decltype(set_tag)::value;
#pragma unroll
        for (int i = 0; i < KV; ++i)
        {
            const uint32_t v = tid + 256 * i, key = v / (HD / 8), ch = v % (HD / 8);
            kr[SI][i] = *(const u32x4 *)(Kh + (size_t)min(jb + key, kv - 1) * HD + ch * 8);
        }
    };
    auto store_k = [&](auto set_tag, int buf) {
        constexpr int SI = decltype(set_tag)::value;
#pragma unroll
        for (int i = 0; i < KV; ++i)
        {
            const uint32_t v = tid + 256 * i, key = v / (HD / 8), ch = v % (HD / 8);
            *(u32x4 *)(Kt(buf) + key * KROW + ch * 8) = kr[SI][i];
        }
    };
    // S^T of the wave's 16 rows against the block's 64 keys: st[b][e] = score of key 16 b + 4 q4 + e, row c16
    auto scores = [&](int buf, f32x4a *st) {
#pragma unroll
        for (int b = 0; b < 4; ++b)
        {
            st[b] = (f32x4a){0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int ks = 0; ks < KS; ++ks)
            {
                const f16x8a a = *(const f16x8a *)(Kt(buf) + (16 * b + c16) * KROW + ks * 32 + 8 * q4);
                st[b] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, qf[ks], st[b], 0, 0, 0);
            }
#pragma unroll
            for (int e = 0; e < 4; ++e)
                st[b][e] = h2f(f2h(st[b][e] * scale));
        }
    };

    // ---- pass 1: row max over all kv positions, sum of exp over the causal ones
    // The wave's rows span positions [pos_lo, pos_hi]: a block wholly before pos_lo (and inside kv) needs no masks,
    // and a block wholly after pos_hi adds nothing to the sums, only to the max.
    const uint32_t pos_lo = offset + min(row0 + wave * 16, S - 1), pos_hi = offset + min(row0 + wave * 16 + 15, S - 1);
    if constexpr (ONE)
    {
        // kv <= 128: every K and V row of the step in one round trip (V blocks 0 and 1 are in flight since entry),
        // all four tiles in LDS behind one barrier, and each block's scores kept in registers from the statistics to
        // the probabilities, so nothing is computed twice. The statistics and the probabilities are the arithmetic
        // of the two passes below (pass 1's step1, pass 2's step2) in the same order, so the outputs are the same
        // bit for bit.
        const uint32_t nb = (kv + kPfKeys - 1) / kPfKeys; // 1 or 2 (the launcher's condition)
        const uint32_t last = offset + min(row0 + kPfRows, S) - 1, nbp = last / kPfKeys + 1;
        auto store_v1 = [&](auto set_tag, int buf) {
            constexpr int SI = decltype(set_tag)::value;
            if (!transposed)
            {
#pragma unroll
                for (int i = 0; i < VP; ++i)
                {
                    const uint32_t v = tid + 256 * i, p = v % 32, ch = v / 32;
                    const uint32_t col = (((p >> 1) ^ ((tid >> 5) & 1u)) << 2) + 2 * (p & 1);
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                    {
                        uint16_t *row = Vt(buf) + (8 * ch + 2 * e) * VROW + col;
                        *(uint32_t *)row = (vr[SI][i][e] & 0xffffu) | (vr[SI][VP + i][e] << 16);
                        *(uint32_t *)(row + VROW) = (vr[SI][i][e] >> 16) | (vr[SI][VP + i][e] & 0xffff0000u);
                    }
                }
            }
            else
            {
#pragma unroll
                for (int i = 0; i < VT; ++i)
                {
                    const uint32_t v = tid + 256 * i, n = v / (kPfKeys / 8), c = v % (kPfKeys / 8);
                    const u32x4 x = vr[SI][i];
                    *(u32x4 *)(Vt(buf) + n * VROW + 8 * c) = ((tid >> 6) & 1u) ? u32x4{x[2], x[3], x[0], x[1]} : x;
                }
            }
        };
        load_k(S0{}, 0);
        load_k(S1{}, kPfKeys);
        store_k(S0{}, 0);
        store_k(S1{}, 1);
        store_v1(S0{}, 0);
        store_v1(S1{}, 1);
        __syncthreads();
        float m = -FLT_MAX, l = 0.f;
        auto stats = [&](const f32x4a *st, uint32_t jb) {
            const bool inside = jb + kPfKeys <= kv;
            float bm = -FLT_MAX;
#pragma unroll
            for (int b = 0; b < 4; ++b)
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    if (inside || jb + 16 * b + 4 * q4 + e < kv)
                        bm = fmaxf(bm, st[b][e]);
            const float mn = fmaxf(m, row4_max(bm));
            float add = 0.f;
            if (jb + kPfKeys <= pos_lo + 1)
            {
                const float nm = -mn * kLog2e;
#pragma unroll
                for (int b = 0; b < 4; ++b)
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        add += pf_exp2(fmaf(st[b][e], kLog2e, nm));
            }
            else if (jb <= pos_hi)
            {
                const float nm = -mn * kLog2e;
#pragma unroll
                for (int b = 0; b < 4; ++b)
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        if (jb + 16 * b + 4 * q4 + e <= pos)
                            add += pf_exp2(fmaf(st[b][e], kLog2e, nm));
            }
            l = l * pf_exp2((m - mn) * kLog2e) + add;
            m = mn;
        };
        f32x4a st0[4], st1[4];
        scores(0, st0);
        stats(st0, 0);
        if (nb > 1)
        {
            scores(1, st1);
            stats(st1, kPfKeys);
        }
        const float inv_l = 1.0f / row4_sum(l), nM = -m * kLog2e;
        f32x4a o[DB];
#pragma unroll
        for (int d = 0; d < DB; ++d)
            o[d] = (f32x4a){0.f, 0.f, 0.f, 0.f};
        const uint32_t vcol = 4 * (q4 ^ ((c16 >> 3) & 1u));
        auto pv = [&](const f32x4a *st, int buf, uint32_t jb) {
            _Float16 ph[4][4];
            const bool full = jb + kPfKeys <= pos_lo + 1;
#pragma unroll
            for (int b = 0; b < 4; ++b)
#pragma unroll
                for (int e = 0; e < 4; ++e)
                {
                    const bool live = full || jb + 16 * b + 4 * q4 + e <= pos;
                    const uint16_t p = f2h(pf_exp2(fmaf(st[b][e], kLog2e, nM)) * inv_l);
                    _Float16 f;
                    __builtin_memcpy(&f, &p, 2);
                    ph[b][e] = live ? f : (_Float16)0.f;
                }
#pragma unroll
            for (int t = 0; t < 2; ++t)
            {
                const f16x8a pb = {ph[2 * t][0],     ph[2 * t][1],     ph[2 * t][2],     ph[2 * t][3],
                                   ph[2 * t + 1][0], ph[2 * t + 1][1], ph[2 * t + 1][2], ph[2 * t + 1][3]};
#pragma unroll
                for (int d = 0; d < DB; ++d)
                {
                    const uint16_t *vp = Vt(buf) + (16 * d + c16) * VROW + 32 * t + vcol;
                    const uint2 lo = *(const uint2 *)vp, hi = *(const uint2 *)(vp + 16);
                    f16x8a a;
                    const u32x4 w = {lo.x, lo.y, hi.x, hi.y};
                    __builtin_memcpy(&a, &w, 16);
                    o[d] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, pb, o[d], 0, 0, 0);
                }
            }
        };
        pv(st0, 0, 0);
        if (nbp > 1)
            pv(st1, 1, kPfKeys);
        const uint32_t row = row0 + wave * 16 + c16;
        if (row < S)
        {
            uint16_t *orow = out + (size_t)row * D + (size_t)h * HD;
#pragma unroll
            for (int d = 0; d < DB; ++d)
            {
                const uint2 w = {pack2(f2h(o[d][0]), f2h(o[d][1])), pack2(f2h(o[d][2]), f2h(o[d][3]))};
                const uint32_t col = h * HD + 16 * d + 4 * q4;
                uint16_t *dst = xt ? out + (size_t)xt_vec(row, col / 8) * 8 + col % 8 : orow + 16 * d + 4 * q4;
                *(uint2 *)dst = w;
            }
        }
        return;
    }
    float m = -FLT_MAX, l = 0.f;
    const uint32_t nb1 = (kv + kPfKeys - 1) / kPfKeys;
    // kv <= 2 blocks: pass 1 leaves K blocks 0 and 1 in LDS buffers 0 and 1, where pass 2 reads them; otherwise pass
    // 1's last step requests them again (both register sets are free by then)
    const bool reuse_k = nb1 <= 2;
    auto step1 = [&](auto ld, auto cur, auto nxt, int buf, uint32_t jb) {
        if constexpr (decltype(ld)::value >= 1)
            load_k(cur, jb + 2 * kPfKeys);
        if constexpr (decltype(ld)::value < 0)
            if (!reuse_k)
            {
                load_k(S0{}, 0);
                load_k(S1{}, kPfKeys);
            }
        f32x4a st[4];
        scores(buf, st);
        const bool inside = jb + kPfKeys <= kv;
        float bm = -FLT_MAX;
#pragma unroll
        for (int b = 0; b < 4; ++b)
#pragma unroll
            for (int e = 0; e < 4; ++e)
                if (inside || jb + 16 * b + 4 * q4 + e < kv)
                    bm = fmaxf(bm, st[b][e]);
        const float mn = fmaxf(m, row4_max(bm));
        float add = 0.f;
        if (jb + kPfKeys <= pos_lo + 1)
        {
            const float nm = -mn * kLog2e;
#pragma unroll
            for (int b = 0; b < 4; ++b)
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    add += pf_exp2(fmaf(st[b][e], kLog2e, nm));
        }
        else if (jb <= pos_hi)
        {
            const float nm = -mn * kLog2e;
#pragma unroll
            for (int b = 0; b < 4; ++b)
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    if (jb + 16 * b + 4 * q4 + e <= pos)
                        add += pf_exp2(fmaf(st[b][e], kLog2e, nm));
        }
        l = l * pf_exp2((m - mn) * kLog2e) + add;
        m = mn;
        if constexpr (decltype(ld)::value >= 0)
        {
            store_k(nxt, buf ^ 1);
            __syncthreads();
        }
    };
    // LD: the step requests block + 2 (1), only stores the next block (0), or neither (-1): the last two steps of a
    // pass request nothing past it, so the next pass does not wait behind loads it never uses (pass 1's last step
    // requests pass 2's first K blocks instead)
    using Ld = std::integral_constant<int, 1>;
    using St = std::integral_constant<int, 0>;
    using Nn = std::integral_constant<int, -1>;
    const uint32_t nb1e = (nb1 + 1) & ~1u;
    load_k(S0{}, 0);
    load_k(S1{}, kPfKeys);
    store_k(S0{}, 0);
    __syncthreads();
    uint32_t blk = 0;
    for (; blk + 2 < nb1e; blk += 2)
    {
        step1(Ld{}, S0{}, S1{}, 0, blk * kPfKeys);
        step1(Ld{}, S1{}, S0{}, 1, (blk + 1) * kPfKeys);
    }
    if (blk + 1 < nb1)
    {
        step1(St{}, S0{}, S1{}, 0, blk * kPfKeys);
        step1(Nn{}, S1{}, S0{}, 1, (blk + 1) * kPfKeys);
    }
    else
        step1(Nn{}, S0{}, S1{}, 0, blk * kPfKeys);
    __syncthreads(); // the last block's LDS reads are done before pass 2 stores into that buffer
    const float M = m, L = row4_sum(l), inv_l = 1.0f / L, nM = -M * kLog2e;

    // ---- pass 2: probabilities and P.V over the blocks at or before the workgroup's last row
    const uint32_t last = offset + min(row0 + kPfRows, S) - 1;
    const uint32_t nb2 = last / kPfKeys + 1;
    f32x4a o[DB];
#pragma unroll
    for (int d = 0; d < DB; ++d)
        o[d] = (f32x4a){0.f, 0.f, 0.f, 0.f};
    auto store_v = [&](auto set_tag, int buf) {
        constexpr int SI = decltype(set_tag)::value;
        if (!transposed)
        {
#pragma unroll
            for (int i = 0; i < VP; ++i)
            {
                // rows 8 ch + 2 e (+ 1) swizzle by ch & 1 = (tid / 32) & 1 (256 i / 32 is even)
                const uint32_t v = tid + 256 * i, p = v % 32, ch = v / 32;
                const uint32_t col = (((p >> 1) ^ ((tid >> 5) & 1u)) << 2) + 2 * (p & 1);
#pragma unroll
                for (int e = 0; e < 4; ++e)
                {
                    uint16_t *row = Vt(buf) + (8 * ch + 2 * e) * VROW + col;
                    *(uint32_t *)row = (vr[SI][i][e] & 0xffffu) | (vr[SI][VP + i][e] << 16);
                    *(uint32_t *)(row + VROW) = (vr[SI][i][e] >> 16) | (vr[SI][VP + i][e] & 0xffff0000u);
                }
            }
        }
        else
        {
#pragma unroll
            for (int i = 0; i < VT; ++i)
            {
                const uint32_t v = tid + 256 * i, n = v / (kPfKeys / 8), c = v % (kPfKeys / 8);
                // units 2c and 2c + 1 trade places in the rows that swizzle ((n >> 3) & 1 = (tid >> 6) & 1)
                const u32x4 x = vr[SI][i];
                *(u32x4 *)(Vt(buf) + n * VROW + 8 * c) = ((tid >> 6) & 1u) ? u32x4{x[2], x[3], x[0], x[1]} : x;
            }
        }
    };
    const uint32_t vcol = 4 * (q4 ^ ((c16 >> 3) & 1u));
    auto step2 = [&](auto ld, auto cur, auto nxt, int buf, uint32_t jb) {
        if constexpr (decltype(ld)::value >= 1)
        {
            load_k(cur, jb + 2 * kPfKeys);
            load_v(cur, jb + 2 * kPfKeys);
        }
        f32x4a st[4];
        scores(buf, st);
        _Float16 ph[4][4];
        const bool full = jb + kPfKeys <= pos_lo + 1;
#pragma unroll
        for (int b = 0; b < 4; ++b)
#pragma unroll
            for (int e = 0; e < 4; ++e)
            {
                const bool live = full || jb + 16 * b + 4 * q4 + e <= pos;
                const uint16_t p = f2h(pf_exp2(fmaf(st[b][e], kLog2e, nM)) * inv_l);
                _Float16 f;
                __builtin_memcpy(&f, &p, 2);
                ph[b][e] = live ? f : (_Float16)0.f;
            }
#pragma unroll
        for (int t = 0; t < 2; ++t)
        {
            // K slots 8 q4 + i: keys 32 t + 4 q4 + i (i < 4) and 32 t + 16 + 4 q4 + (i - 4)
            const f16x8a pb = {ph[2 * t][0],     ph[2 * t][1],     ph[2 * t][2],     ph[2 * t][3],
                               ph[2 * t + 1][0], ph[2 * t + 1][1], ph[2 * t + 1][2], ph[2 * t + 1][3]};
#pragma unroll
            for (int d = 0; d < DB; ++d)
            {
                // row 16 d + c16 swizzles by (c16 >> 3) & 1: unit 8 t + q4 (+ 4) sits at 8 t + (q4 ^ that) (+ 4)
                const uint16_t *vr = Vt(buf) + (16 * d + c16) * VROW + 32 * t + vcol;
                const uint2 lo = *(const uint2 *)vr, hi = *(const uint2 *)(vr + 16);
                f16x8a a;
                const u32x4 w = {lo.x, lo.y, hi.x, hi.y};
                __builtin_memcpy(&a, &w, 16);
                o[d] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, pb, o[d], 0, 0, 0);
            }
        }
        if constexpr (decltype(ld)::value >= 0)
        {
            if (!reuse_k) // nb2 <= nb1, so with reuse_k this is block 1, already in buffer 1
                store_k(nxt, buf ^ 1);
            store_v(nxt, buf ^ 1);
            __syncthreads();
        }
    };
    const uint32_t nb2e = (nb2 + 1) & ~1u;
    // blocks 0 and 1 are in flight (V since entry, K since pass 1's last step) or, with reuse_k, K is in LDS
    if (!reuse_k)
        store_k(S0{}, 0);
    store_v(S0{}, 0);
    __syncthreads();
    for (blk = 0; blk + 2 < nb2e; blk += 2)
    {
        step2(Ld{}, S0{}, S1{}, 0, blk * kPfKeys);
        step2(Ld{}, S1{}, S0{}, 1, (blk + 1) * kPfKeys);
    }
    if (blk + 1 < nb2)
    {
        step2(St{}, S0{}, S1{}, 0, blk * kPfKeys);
        step2(Nn{}, S1{}, S0{}, 1, (blk + 1) * kPfKeys);
    }
    else
        step2(Nn{}, S0{}, S1{}, 0, blk * kPfKeys);
    // O^T accumulators: o[d][e] = out[row c16][dim 16 d + 4 q4 + e]
    const uint32_t row = row0 + wave * 16 + c16;
    if (row < S)
    {
        uint16_t *orow = out + (size_t)row * D + (size_t)h * HD;
#pragma unroll
        for (int d = 0; d < DB; ++d)
        {
            const uint2 w = {pack2(f2h(o[d][0]), f2h(o[d][1])), pack2(f2h(o[d][2]), f2h(o[d][3]))};
            // column h HD + 16 d + 4 q4: in fragment order the 4 halfs sit in the second half of vector kv when q4 is
            // odd
            const uint32_t col = h * HD + 16 * d + 4 * q4;
            uint16_t *dst = xt ? out + (size_t)xt_vec(row, col / 8) * 8 + col % 8 : orow + 16 * d + 4 * q4;
            *(uint2 *)dst = w;
        }
    }
}

// LDS of the kernel: two K tiles [key][dim] (pf_krow pitch) and two V tiles [dim][key] (rows padded by 8 halves)
template <int HD> constexpr size_t pf_lds_bytes()
{
    return (size_t)2 * (kPfKeys * pf_krow<HD>() + HD * (kPfKeys + 8)) * sizeof(uint16_t);
}

template <int HD, bool ONE>
static hipError_t launch_pf_hd(hipStream_t st, dim3 grid, const uint16_t *q, const uint16_t *kc, const uint16_t *vc,
                               uint16_t *out, uint32_t offset, uint32_t S, uint32_t H, uint32_t ctx, float scale,
                               bool xt)
{
    static uint64_t attr_devs = 0; // devices on which the LDS limit is raised for this kernel
    constexpr size_t lds = pf_lds_bytes<HD>();
    hipError_t e = lds_attr_once((const void *)attn_prefill_mfma_kernel<HD, ONE>, lds, attr_devs);
    if (e != hipSuccess)
        return e;
    attn_prefill_mfma_kernel<HD, ONE><<<grid, 256, lds, st>>>(q, kc, vc, out, offset, S, H, ctx, scale, xt);
    return hipGetLastError();
}

bool attn_prefill_mfma_ok(uint32_t hd)
{
    return hd == 64 || hd == 128;
}

hipError_t launch_attn_prefill_mfma(hipStream_t st, const uint16_t *q, const uint16_t *kc, const uint16_t *vc,
                                    uint16_t *out, uint32_t offset, uint32_t S, uint32_t H, uint32_t hd, uint32_t ctx,
                                    float scale, bool xt)
{
    if (S == 0 || offset + S > ctx || !attn_prefill_mfma_ok(hd) || (xt && S > 128))
        return hipErrorInvalidValue;
    const dim3 grid(H, (S + kPfRows - 1) / kPfRows);
    // a step whose kv fits two key blocks takes the one-pass form (its own instantiation, so the two-pass kernel's
    // code and registers are those it has without it)
    const bool one = offset + S <= 2 * kPfKeys;
    if (hd == 128)
        return one ? launch_pf_hd<128, true>(st, grid, q, kc, vc, out, offset, S, H, ctx, scale, xt)
                   : launch_pf_hd<128, false>(st, grid, q, kc, vc, out, offset, S, H, ctx, scale, xt);
    return one ? launch_pf_hd<64, true>(st, grid, q, kc, vc, out, offset, S, H, ctx, scale, xt)
               : launch_pf_hd<64, false>(st, grid, q, kc, vc, out, offset, S, H, ctx, scale, xt);
}

} // namespace vk
