// Launchers of the gfx950 kernels. Internal to libvkllm; every launcher enqueues on `stream` and returns the
// launch status. Tensor views carry ELEMENT strides.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace vk
{

enum DType : int32_t
{
    DT_F32 = 1,
    DT_F16 = 2,
    DT_I8 = 3,
    DT_U32 = 4
};

struct TView
{
    void *p;
    uint32_t n[4]; // shapes [N, C, H, W]
    uint32_t s[4]; // element strides
    int32_t dt;
};

// ---- generic operators (node-by-node execution and the op API) ----
hipError_t launch_copy(hipStream_t st, const TView &in, const TView &out);
hipError_t launch_bin(hipStream_t st, const TView &a, const TView &b, const TView &out, int op);
hipError_t launch_embedding(hipStream_t st, const TView &idx, const TView &table, const TView &out, uint32_t unk);
hipError_t launch_rmsnorm(hipStream_t st, const TView &x, const TView &w, const TView &out, float eps);
// out = act(scale * a . b), b [N,K] when transposed_b else [K,N]; size-1 batch dims broadcast
hipError_t launch_matmul(hipStream_t st, const TView &a, const TView &b, const TView &out, float scale, int act,
                         bool transposed_b);
// freqs_host[w] = base^(2w/D) for w < D/2 (D <= 2*kMaxRopeFreqs), passed by value in the kernel arguments
constexpr int kMaxRopeFreqs = 256;
hipError_t launch_rope(hipStream_t st, const TView &in, const TView &out, uint32_t offset, const float *freqs_host,
                       bool neox);
hipError_t launch_softmax(hipStream_t st, const TView &in, const TView &out, int seq_mask, uint32_t offsets);
hipError_t launch_update_rows(hipStream_t st, const TView &src, const TView &cache, uint32_t offset_rows);
hipError_t launch_arg_max(hipStream_t st, const TView &in, const TView &out);
hipError_t launch_ffn_up_and_gate(hipStream_t st, const TView &x, const TView &wu, const TView &wg, const TView &out);

// ---- fused LLaMA-2 token step ----
// Device-resident step parameters, read by the kernels so a captured decode graph replays for any position.
struct Step
{
    uint32_t offset; // position of the step's first token
    uint32_t S;      // tokens in the step
};

// Inputs and output of a single-token step in pinned host memory: the host writes the position and token before
// the step, the first kernel copies them into the device Step, the arg max writes the chosen id back.
struct DecodeIo
{
    uint32_t offset;
    uint32_t token;
    uint32_t id;
    uint32_t err;       // nonzero when a kernel's bounded wait gave up during the step
    uint32_t token_dev; // nonzero: the step's token is the device-side arg max of the step before (launch-ahead)
};
// single-token step: step = {io->offset, 1}, h = embd[token] (ids >= V read row unk), where token is io->token, or
// *prev_id when io->token_dev is set
hipError_t launch_embed_decode(hipStream_t st, const DecodeIo *io, Step *step, const uint16_t *embd, uint16_t *h,
                               uint32_t V, uint32_t D, uint32_t unk, const uint32_t *prev_id);
// h[s] = embd[toks[s]] (ids >= V read row unk), s < S; D % 8 == 0
hipError_t launch_embed_rows(hipStream_t st, const uint32_t *toks, uint32_t S, const uint16_t *embd, uint16_t *h,
                             uint32_t V, uint32_t D, uint32_t unk);
// y[s] = rmsnorm(x[s]) * w, s < S; with xt, y is fragment-ordered (xt_vec; S <= 128, D % 16 == 0)
hipError_t launch_rmsnorm_rows(hipStream_t st, const uint16_t *x, const float *w, uint16_t *y, uint32_t S,
                               uint32_t D, float eps, bool xt = false);

enum GemvEpi : int
{
    EPI_PLAIN = 0, // out[r] = fp16(acc_r)
    EPI_RESID = 1, // out[r] = fp16(resid[r] + fp16(acc_r)), in place allowed
    EPI_GATEUP = 2, // rows [0,F) up, [F,2F) gate: out[r] = fp16(fp16(up_r) * fp16(silu(gate_r)))
    EPI_QKV = 3,   // rows [0,3D) of [Wq;Wk;Wv]: RoPE on q,k; q -> out, k/v -> caches at step->offset
    // EPI_PLAIN's out, and the arg max of all rows under the reference's order (am_before) into am_ids[0] and
    // am_io->id: each workgroup publishes its best (value, row), the last to arrive on the am_count counters
    // reduces them and clears the counters (no workgroup waits for another)
    EPI_ARGMAX = 4,
    EPI_RAW = 5, // EPI_PLAIN's out from the input as given, no RMSNorm (the MATMUL op's mat_mul_vec case)
    // EPI_QKV, then each head's single-token attention (kv = step->offset + 1 <= kAttnTailMaxKv) computed by the
    // workgroup that completes the head's q, k and v rows: attn_out[h*hd + d] as the short-cache attention kernel
    // leaves it. head_count [H] counts completed units per head (zero between launches).
    EPI_QKV_ATTN = 6,
};
// the decode QKV product's attention tail: heads at most, and positions at most (its scores and partial sums reuse
// the GEMV's input LDS, sized to hold kAttnTailMaxKv + 4 * hd floats)
constexpr uint32_t kAttnTailMaxHeads = 64, kAttnTailMaxKv = 512;

struct GemvArgs
{
    const uint16_t *x;      // input vector [K] (the residual stream when norm_w is set)
    const float *norm_w;    // RMSNorm weight: x is normalised in the prologue; nullptr: x used as is
    float eps;
    const uint16_t *w;      // weight rows [rows, K], K contiguous
    uint32_t K;
    uint32_t units;         // fallback kernel (K > 14336) work units: PLAIN/RESID ceil(rows/2), GATEUP F, QKV 3D/2
    uint32_t rows_per_unit; // rows a wave reduces at once (1, 2 or 4); 0 picks the default for the shape
    uint32_t rows;          // weight rows
    uint16_t *out;
    const uint16_t *resid;  // EPI_RESID
    // EPI_QKV
    uint16_t *kc, *vc;      // layer caches [H, ctx, hd]
    const Step *step;
    const float *freqs;     // base^(2w/hd), w < hd/2
    uint32_t D, hd, ctx;
    // EPI_QKV_ATTN
    uint16_t *attn_out;     // [H, hd]
    uint32_t *head_count;   // [H]
    uint32_t H;
    float attn_scale;
    uint32_t *attn_err;     // set (system scope) when the step's position exceeds kAttnTailMaxKv
    // EPI_ARGMAX (fast kernel only, one row per unit; a launch of more than am_cap workgroups is refused)
    uint32_t *am_ids;   // [1]
    DecodeIo *am_io;    // optional
    float *am_val;      // per-workgroup candidates [am_cap]
    uint32_t *am_idx;   // [am_cap]
    uint32_t *am_count; // arrival counters [kArgmaxSyncWords], zero between launches
    uint32_t am_cap;
};
// EPI_ARGMAX arrival counters: kArgmaxCounters first-level words and one top word, each on its own 256 bytes
constexpr uint32_t kArgmaxCounters = 16, kArgmaxStride = 64, kArgmaxSyncWords = (kArgmaxCounters + 1) * kArgmaxStride;
hipError_t launch_gemv(hipStream_t st, int epi, const GemvArgs &a, int cu_count);

// Single-token attention over the cache for every head (kv = step->offset + 1): s_j = fp16(scale q.k_j),
// p = fp16(softmax(s)), out[h*hd + d] = fp16(sum_j p_j v_j[d]); when kv == hd the product is p . V^T (the
// reference's shape-based transposition rule). Long caches: attn_scores splits the keys into `cmax` chunks of
// `chunk` positions (chunk * cmax >= ctx), attn_pv forms each chunk's partial sums and merges them.
// Short caches: attn_small does it all in one kernel (`groups` slices of the head's dims, each scoring all keys).
struct AttnDecodeArgs
{
    const uint16_t *q;        // [H, hd]
    const uint16_t *kc, *vc;  // [H, ctx, hd]
    uint16_t *out;            // [H, hd]
    const Step *step;
    float *scores;            // [H, ctx]
    float *stats;             // [H, cmax, 2]: chunk max, chunk sum of exp
    float *part;              // [H, cmax, hd]: chunk partial sums
    uint32_t *count;          // [H]: chunk arrivals, zero before the first launch; the kernels leave it zero
    uint32_t H, hd, ctx, cmax, chunk, groups;
    float scale;
    uint32_t small_max; // one-kernel attention: positions its LDS holds (set by the launchers)
    // one-kernel long-cache attention: [H * kAttnLongStride] per-head counters, zero before the first launch (the
    // kernel leaves them zero), and the flag it sets (system scope) when a wait gives up
    uint32_t *long_sync;
    uint32_t *err;
    // polls a bounded wait makes before it gives up (the one-kernel long-cache attention and the attention +
    // projection launch); 0 gives up at once, without polling, so the failure path can be forced from the host
    uint32_t spin_limit;
};
constexpr uint32_t kAttnLongStride = 64;
// default spin limits of the bounded waits: each poll sleeps ~64 clocks, so these are ~0.5 s and ~0.1 s
constexpr uint32_t kAttnLongSpinLimit = 1u << 20;
constexpr uint32_t kAttnOSpinLimit = 1u << 18;
// dim slices per head: the largest divisor of hd / 8 up to max_groups with H * groups <= 1024
uint32_t attn_groups(uint32_t H, uint32_t hd, uint32_t max_groups);
hipError_t launch_attn_scores(hipStream_t st, const AttnDecodeArgs &a);
hipError_t launch_attn_pv(hipStream_t st, const AttnDecodeArgs &a);
// Long caches in one launch: block (h, c) scores its chunk, publishes the chunk's statistics, waits for the other
// chunks of head h, then forms its partial sums as attn_pv does (identical results). hipErrorInvalidConfiguration
// when the device cannot hold every chunk block at once (then use attn_scores + attn_pv).
hipError_t launch_attn_long(hipStream_t st, const AttnDecodeArgs &a, int cu_count);
// whether launch_attn_long takes this shape (head_dim <= 128, chunks of hd to 256 positions covering ctx); shapes it
// does not take run on attn_scores + attn_pv
bool attn_long_ok(const AttnDecodeArgs &a);
// largest kv the one-kernel attention takes for this shape (0: the shape needs the two-kernel path)
uint32_t attn_small_limit(const AttnDecodeArgs &a);
// kv <= kv_max <= min(ctx, attn_small_limit); kv_max sizes the LDS
hipError_t launch_attn_small(hipStream_t st, const AttnDecodeArgs &a, uint32_t kv_max);

// One-kernel attention followed in the same launch by out[r] = fp16(resid[r] + fp16(Wo[r] . attn)) for r < H*hd
// (K = H*hd); at.out receives the attention output. hipErrorInvalidConfiguration when the device cannot hold the
// attention blocks and projection blocks at once (then launch them separately).
constexpr uint32_t kAttnSyncWords = 1024;
struct AttnOArgs
{
    AttnDecodeArgs at;
    const uint16_t *wo;    // [H*hd, H*hd]
    const uint16_t *resid; // residual stream in
    uint16_t *out;         // residual stream out (may be resid)
    uint32_t *sync;        // [kAttnSyncWords] zero before the first launch; every launch leaves them zero
    uint32_t *err;         // set to 1 (system scope) when a wait gave up
    uint32_t attn_blocks;  // set by the launcher
};
hipError_t launch_attn_o(hipStream_t st, const AttnOArgs &a, uint32_t kv_max, int cu_count);

// ---- persistent single-token step (decode_persist.hip): every layer and the vocabulary product in one launch ----
struct PersistLayer
{
    const uint16_t *wqkv, *wo, *wug, *wd; // [3D, D], [D, D], [2F, D] (up rows, then gate rows), [D, F]
    const float *attn_norm, *ffn_norm;
    uint16_t *kc, *vc; // [H, ctx, hd]
};
struct PersistArgs
{
    const PersistLayer *layers; // [L], device memory
    uint32_t L, D, F, V, H, hd, ctx;
    float eps, scale;
    const Step *step; // the step's position (written by the embedding kernel)
    const float *freqs;
    const float *out_norm;
    const uint16_t *out_w;
    // activations, each row written once per step and read only after it is written: hs [2L + 1][hstride] the
    // residual stream (hs[0] the embedding row, hs[2l + 1] after layer l's attention, hs[2l + 2] after its FFN),
    // qs and attns [L][hstride], acts [L][fstride]; strides in halves, multiples of 128
    uint16_t *hs, *qs, *attns, *acts;
    uint32_t hstride, fstride;
    uint16_t *logits;   // [V]
    uint32_t small_max; // the attention's positions bound (its LDS and speculative cache reads)
    uint32_t *sync;     // kPersistSyncWords, zero before the first launch; every launch leaves them zero
    uint32_t *err;      // set (system scope) when a wait gives up; the step's outputs are then not valid
    uint32_t spin_limit;
    // the arg max (as GemvArgs' EPI_ARGMAX fields)
    uint32_t *am_ids;
    DecodeIo *am_io;
    float *am_val;
    uint32_t *am_idx, *am_count;
    uint32_t am_cap;
};
constexpr uint32_t kPersistSyncWords = 12 * 64;
// hipErrorInvalidValue: a shape without a compiled instantiation, or a positions bound the attention part does not
// take (nothing launched); hipErrorInvalidConfiguration: fewer than one resident workgroup per CU at this LDS size
hipError_t launch_decode_persist(hipStream_t st, const PersistArgs &a, int cu_count);

// prefill: queries s < S at positions offset+s attend to positions <= offset+s (the row max over all offset+S);
// head sizes 64 and 128 run on the MFMA kernel, others one workgroup per (row, head)
bool attn_prefill_mfma_ok(uint32_t hd);
// with xt, out is fragment-ordered (xt_vec; S <= 128)
hipError_t launch_attn_prefill_mfma(hipStream_t st, const uint16_t *q, const uint16_t *kc, const uint16_t *vc,
                                    uint16_t *out, uint32_t offset, uint32_t S, uint32_t H, uint32_t hd, uint32_t ctx,
                                    float scale, bool xt = false);
hipError_t launch_attn_prefill(hipStream_t st, const uint16_t *q, const uint16_t *kc, const uint16_t *vc,
                               uint16_t *out, uint32_t offset, uint32_t S, uint32_t H, uint32_t hd, uint32_t ctx,
                               float scale, bool xt = false);
// qkv [S, 3D] -> RoPE'd q [S, D]; RoPE'd k and v into the caches at rows offset..offset+S-1
hipError_t launch_rope_kv(hipStream_t st, const uint16_t *qkv, uint16_t *q, uint16_t *kc, uint16_t *vc,
                          const float *freqs, uint32_t offset, uint32_t S, uint32_t D, uint32_t hd, uint32_t ctx);
// act[s][n] = fp16(ug[s][n] * ug[s][F + n])
hipError_t launch_swiglu(hipStream_t st, const uint16_t *ug, uint16_t *act, uint32_t S, uint32_t F);
// ids[s] = arg_max(logits[s]) with the reference's tie rule, contiguous rows of V; with `io`, row 0's id also goes
// to io->id
hipError_t launch_argmax_rows(hipStream_t st, const uint16_t *logits, uint32_t *ids, uint32_t S, uint32_t V,
                              DecodeIo *io = nullptr);

enum GemmEpi : int
{
    GEMM_PLAIN = 0,   // C = fp16(acc)
    GEMM_SILU_HI = 1, // columns >= split: fp16(silu(acc)), others fp16(acc)
    GEMM_RESID = 2,   // C = fp16(C + fp16(acc)) (C holds the residual)
    // B = [Wu; Wg] (split = F rows each, N = 2F, F % 32 == 0, K % 64 == 0): C[m][f] (f < F, row stride ldc) =
    // fp16(fp16(A[m] . Wu[f]) * fp16(silu(A[m] . Wg[f]))). The product reads B's rows as interleaved 32-row blocks
    // of up and gate rows, so both values of an output meet in one lane.
    GEMM_SWIGLU = 3,
    // B = [Wq; Wk; Wv] (N = 3D, D % 64 == 0, K % 64 == 0, head size a power of two >= 32): the product's row m
    // (position rope.offset + m) goes out
    // as the prompt step's q, k and v: q and k rotated by RoPE (each element first rounded to fp16, then the
    // rotation of launch_rope_kv), q -> rope.q[m][c], k and v -> the caches at that position; C is not written
    GEMM_QKV_ROPE = 4,
};
struct GemmRope
{
    uint16_t *q;         // [M, D]
    uint16_t *kc, *vc;   // layer caches [H, ctx, hd]
    const float *cs;     // [M][hd / 2][2]: cos and sin of (offset + m) / base^(2w/hd), from launch_rope_table
    uint32_t offset, D, hd, ctx;
};
// GEMM_RESID followed by y[m] = RMSNorm(C[m]) * w (ldc == N; the norm of launch_rmsnorm_rows); with xt, y is
// fragment-ordered (xt_vec; M <= 128)
struct GemmNorm
{
    const float *w;
    uint16_t *y;
    float eps;
    bool xt = false;
};
// C[M, N] (row stride ldc) = A[M, K] . B[N, K]^T, fp16 operands, fp32 accumulation on MFMA. K % 8 == 0.
// `work` (work_elems floats) holds split-K partial tiles for short prompts; with too little of it K is not split.
// `rope` is read by GEMM_QKV_ROPE only; `norm` (GEMM_RESID only) adds the RMSNorm of the updated rows, fused into
// the split-K reduce when K is split.
hipError_t launch_gemm(hipStream_t st, int epi, const uint16_t *A, const uint16_t *B, uint16_t *C, uint32_t M,
                       uint32_t N, uint32_t K, uint32_t ldc, uint32_t split, int cu_count, float *work,
                       size_t work_elems, const GemmRope *rope = nullptr, const GemmNorm *norm = nullptr);
// Prompt-step products of at most 128 tokens with the weights read from a fragment-tiled copy (launch_tile_weights)
// and X fragment-ordered (xt_vec): C[M, N] = X[M, K] . W[N, K]^T, M <= 128, K % 16 == 0.
enum StreamEpi : int
{
    STREAM_PARTIAL = 0, // work[z][M][N]: fp32 partials of K range z (N % 32 == 0), for launch_gemm_reduce
    STREAM_PLAIN = 1,   // C[m][n] = fp16(acc), row stride ldc
    STREAM_SWIGLU = 2,  // the interleaved [Wu; Wg] copy (N = 2F): C[m][f] = fp16(fp16(up) * fp16(silu(gate)))
    STREAM_QKV_ROPE = 3, // [Wq; Wk; Wv] (N = 3 rope->D): q rotated into rope->q, k rotated and v into the caches, as
                         // launch_gemm's GEMM_QKV_ROPE; C is not written
};
// halfs of the tiled copy of W [N, K] (F > 0: [Wu; Wg] with N = 2F, F % 16 == 0, rows interleaved in 16s)
size_t stream_tiled_elems(uint32_t N, uint32_t K, uint32_t F);
hipError_t launch_tile_weights(hipStream_t st, const uint16_t *W, uint16_t *Wt, uint32_t N, uint32_t K, uint32_t F);
// row-major X [M <= 128, K] -> fragment order (128 * K halfs, rows past M zero)
hipError_t launch_tile_activations(hipStream_t st, const uint16_t *X, uint16_t *Xt, uint32_t M, uint32_t K);
// *splits: K ranges wanted for STREAM_PARTIAL (0: enough for about one workgroup per CU); on return the ranges used
// (1 for the other epilogues). work holds work_elems floats; rope is STREAM_QKV_ROPE's.
hipError_t launch_stream_gemm(hipStream_t st, int epi, const uint16_t *X, const uint16_t *Wt, uint16_t *C,
                              float *work, size_t work_elems, uint32_t M, uint32_t N, uint32_t K, uint32_t ldc,
                              uint32_t *splits, const GemmRope *rope = nullptr);
// The epilogue of split-K partials work[z][M][N] (z < splits, added in order), as launch_gemm applies it: GEMM_RESID
// (C += the sum; with `norm`, the rows' RMSNorm as well) or GEMM_QKV_ROPE (`rope`'s q and caches).
hipError_t launch_gemm_reduce(hipStream_t st, int epi, const float *work, uint16_t *C, uint32_t M, uint32_t N,
                              uint32_t splits, const GemmRope *rope = nullptr, const GemmNorm *norm = nullptr);
// Looks up the device address of the allocation-free GEMM's scratch array on device `dev` (current), once per
// device; vkllm_context_new calls it.
hipError_t noalloc_scratch_init(int dev);
// cs[s][w] = (cos f, sin f) with f = (offset + s) / freqs[w], s < S, w < hd / 2 (the angles launch_rope_kv uses)
hipError_t launch_rope_table(hipStream_t st, float *cs, const float *freqs, uint32_t offset, uint32_t S,
                             uint32_t hd);

// ---- synthetic weights: dst[i] = fp16(normal(stream, i) * std), i < count ----
hipError_t launch_random_f16(hipStream_t st, uint16_t *dst, uint64_t count, uint64_t stream_key, float std);
hipError_t launch_fill_f32(hipStream_t st, float *dst, uint64_t count, float v);

} // namespace vk
