// Fused execution of a LLaMA-2 token step built by vkllm_models_llama2_build_graph.
//
// The graph keeps the reference's node structure (src/models/vkllm_models_llama2.c:488-602); its plan records
// (model, input ids, offset, S). Running the plan:
//   S == 1  the decode step: embed, 5 fused kernels per layer, logits, arg max. Kernels read the position from a
//           device-resident Step, so the whole sequence is captured once per model as a hipGraph and replayed for
//           every token; only the token id and position are copied in before each replay.
//   S >  1  prefill: embed, per layer RMSNorm -> QKV GEMM (MFMA) -> RoPE + KV append -> attention -> Wo GEMM with
//           the residual add -> RMSNorm -> [up;gate] GEMM with SiLU on the gate half -> up*gate -> Wd GEMM with
//           the residual add; then RMSNorm -> logits GEMM for all S rows -> arg max per row.
// Either way the S arg-max ids land in the mapped output tensor, as the reference's ARG_MAX node leaves them.
#include <cmath>
#include <cstdlib>
#include <cstring>

#include "model_priv.h"

struct FusedPlan
{
    vkllm_models_llama2 *model;
    vkllm_tensor *input_toks;
    uint32_t offset;
    uint32_t S;
};

struct FusedState
{
    uint32_t cap_S = 0; // rows the activation buffers hold
    uint16_t *h = nullptr, *xn = nullptr, *qkv = nullptr, *q = nullptr, *attn = nullptr, *act = nullptr,
             *ug = nullptr, *logits = nullptr;
    uint32_t *ids = nullptr, *toks = nullptr;
    vk::Step *step = nullptr;    // device
    vk::Step *step_h = nullptr;  // pinned staging for step + first token
    uint32_t *io_h = nullptr;    // pinned: [0] token for decode, then ids read back
    float *freqs = nullptr;      // device copy of the RoPE denominators
    hipGraph_t graph = nullptr;
    hipGraphExec_t exec = nullptr;
};

void *fused_plan_new(vkllm_models_llama2 *model, vkllm_tensor *input_toks, uint32_t offset)
{
    auto *p = new FusedPlan();
    p->model = model;
    p->input_toks = input_toks;
    p->offset = offset;
    p->S = input_toks->shapes[3];
    return p;
}

void fused_plan_free(void *plan)
{
    delete (FusedPlan *)plan;
}

static void free_buffers(FusedState *fs)
{
    void *bufs[] = {fs->h, fs->xn, fs->qkv, fs->q, fs->attn, fs->act, fs->ug, fs->logits, fs->ids, fs->toks};
    for (void *b : bufs)
        if (b)
            (void)hipFree(b);
    fs->h = fs->xn = fs->qkv = fs->q = fs->attn = fs->act = fs->ug = fs->logits = nullptr;
    fs->ids = fs->toks = nullptr;
    fs->cap_S = 0;
}

void fused_model_release(vkllm_context *ctx, vkllm_models_llama2 *model)
{
    ModelPriv *mp = model_priv(model);
    if (!mp || !mp->fs)
        return;
    FusedState *fs = mp->fs;
    (void)hipStreamSynchronize(ctx->device->stream);
    if (fs->exec)
        (void)hipGraphExecDestroy(fs->exec);
    if (fs->graph)
        (void)hipGraphDestroy(fs->graph);
    free_buffers(fs);
    if (fs->step)
        (void)hipFree(fs->step);
    if (fs->freqs)
        (void)hipFree(fs->freqs);
    if (fs->step_h)
        (void)hipHostFree(fs->step_h);
    if (fs->io_h)
        (void)hipHostFree(fs->io_h);
    delete fs;
    mp->fs = nullptr;
}

static vkllm_err_t ensure_state(vkllm_context *ctx, ModelPriv *mp, uint32_t S)
{
    if (!mp->fs)
    {
        mp->fs = new FusedState();
        FusedState *fs = mp->fs;
        HIP_TRY(hipMalloc(&fs->step, sizeof(vk::Step)));
        HIP_TRY(hipHostMalloc((void **)&fs->step_h, sizeof(vk::Step), hipHostMallocDefault));
        HIP_TRY(hipMalloc(&fs->freqs, sizeof(float) * (mp->hd / 2 + 1)));
        HIP_TRY(hipMemcpyAsync(fs->freqs, mp->rope_freqs.data(), sizeof(float) * mp->hd / 2, hipMemcpyHostToDevice,
                               ctx->device->stream));
    }
    FusedState *fs = mp->fs;
    if (S <= fs->cap_S)
        return VKLLM_ERR_OK;
    // growing the activation buffers moves them: the captured decode graph refers to the old ones
    HIP_TRY(hipStreamSynchronize(ctx->device->stream));
    if (fs->exec)
    {
        (void)hipGraphExecDestroy(fs->exec);
        fs->exec = nullptr;
    }
    if (fs->graph)
    {
        (void)hipGraphDestroy(fs->graph);
        fs->graph = nullptr;
    }
    free_buffers(fs);
    if (fs->io_h)
    {
        (void)hipHostFree(fs->io_h);
        fs->io_h = nullptr;
    }
    const size_t D = mp->D, F = mp->F, V = mp->V, Sz = S;
    HIP_TRY(hipMalloc(&fs->h, Sz * D * 2));
    HIP_TRY(hipMalloc(&fs->xn, Sz * D * 2));
    HIP_TRY(hipMalloc(&fs->qkv, Sz * 3 * D * 2));
    HIP_TRY(hipMalloc(&fs->q, Sz * D * 2));
    HIP_TRY(hipMalloc(&fs->attn, Sz * D * 2));
    HIP_TRY(hipMalloc(&fs->act, Sz * F * 2));
    HIP_TRY(hipMalloc(&fs->ug, Sz * 2 * F * 2));
    HIP_TRY(hipMalloc(&fs->logits, Sz * V * 2));
    HIP_TRY(hipMalloc(&fs->ids, Sz * 4));
    HIP_TRY(hipMalloc(&fs->toks, Sz * 4));
    HIP_TRY(hipHostMalloc((void **)&fs->io_h, Sz * 4, hipHostMallocDefault));
    fs->cap_S = S;
    return VKLLM_ERR_OK;
}

#define KTRY(_ctx, _kid, _call)                                                                                     \
    do                                                                                                              \
    {                                                                                                               \
        hipError_t _e = timed((_ctx), pipeline_of((_ctx), (_kid)), [&]() { return (_call); });                     \
        if (_e != hipSuccess)                                                                                       \
            return hip_fail(_e, #_call, __FILE__, __LINE__);                                                        \
    } while (0)

// RMSNorm(h) -> [Wu;Wg] GEMV -> up * silu(gate) into act, for layer l of a decode step
static vk::GemvArgs gateup_args(const ModelPriv *mp, uint32_t l)
{
    vk::GemvArgs gu{};
    gu.x = mp->fs->h;
    gu.norm_w = mp->layers[l].ffn_norm;
    gu.eps = mp->eps;
    gu.w = mp->layers[l].wug;
    gu.K = mp->D;
    gu.rows = 2 * mp->F;
    gu.units = mp->F;
    gu.out = mp->fs->act;
    return gu;
}

// decode: S == 1, position from fs->step
static vkllm_err_t enqueue_decode(vkllm_context *ctx, ModelPriv *mp)
{
    FusedState *fs = mp->fs;
    hipStream_t st = ctx->device->stream;
    const int cu = ctx->device->cu_count;
    const uint32_t D = mp->D, F = mp->F, V = mp->V, hd = mp->hd;
    const float scale = 1.0f / sqrtf((float)hd);
    KTRY(ctx, KID_F_EMBED, vk::launch_embed_rows(st, fs->toks, 1, mp->embd, fs->h, V, D, mp->pad_id));
    for (uint32_t l = 0; l < mp->L; ++l)
    {
        const ModelPriv::Layer &ly = mp->layers[l];
        vk::GemvArgs g{};
        g.x = fs->h;
        g.norm_w = ly.attn_norm;
        g.eps = mp->eps;
        g.w = ly.wqkv;
        g.K = D;
        g.rows = 3 * D;
        g.units = 3 * D / 2;
        g.out = fs->q;
        g.kc = ly.kc;
        g.vc = ly.vc;
        g.step = fs->step;
        g.freqs = fs->freqs;
        g.D = D;
        g.hd = hd;
        g.ctx = mp->ctx;
        KTRY(ctx, KID_F_QKV, vk::launch_gemv(st, vk::EPI_QKV, g, cu));
        KTRY(ctx, KID_F_ATTN_SCORES,
             vk::launch_attn_decode(st, fs->q, ly.kc, ly.vc, fs->attn, fs->step, mp->H, hd, mp->ctx, scale));
        vk::GemvArgs o{};
        o.x = fs->attn;
        o.w = ly.wo;
        o.K = D;
        o.rows = D;
        o.units = (D + 1) / 2;
        o.out = fs->h;
        o.resid = fs->h;
        KTRY(ctx, KID_F_O_RESID, vk::launch_gemv(st, vk::EPI_RESID, o, cu));
        KTRY(ctx, KID_F_GATEUP, vk::launch_gemv(st, vk::EPI_GATEUP, gateup_args(mp, l), cu));
        vk::GemvArgs dn{};
        dn.x = fs->act;
        dn.w = ly.wd;
        dn.K = F;
        dn.rows = D;
        dn.units = (D + 1) / 2;
        dn.out = fs->h;
        dn.resid = fs->h;
        KTRY(ctx, KID_F_DOWN_RESID, vk::launch_gemv(st, vk::EPI_RESID, dn, cu));
    }
    vk::GemvArgs lg{};
    lg.x = fs->h;
    lg.norm_w = mp->out_norm;
    lg.eps = mp->eps;
    lg.w = mp->out_w;
    lg.K = D;
    lg.rows = V;
    lg.units = (V + 1) / 2;
    lg.out = fs->logits;
    KTRY(ctx, KID_F_LOGITS, vk::launch_gemv(st, vk::EPI_PLAIN, lg, cu));
    KTRY(ctx, KID_F_ARGMAX, vk::launch_argmax_rows(st, fs->logits, fs->ids, 1, V));
    return VKLLM_ERR_OK;
}

static vkllm_err_t enqueue_prefill(vkllm_context *ctx, ModelPriv *mp, uint32_t S, uint32_t offset)
{
    FusedState *fs = mp->fs;
    hipStream_t st = ctx->device->stream;
    const int cu = ctx->device->cu_count;
    const uint32_t D = mp->D, F = mp->F, V = mp->V, hd = mp->hd;
    const float scale = 1.0f / sqrtf((float)hd);
    KTRY(ctx, KID_F_EMBED, vk::launch_embed_rows(st, fs->toks, S, mp->embd, fs->h, V, D, mp->pad_id));
    for (uint32_t l = 0; l < mp->L; ++l)
    {
        const ModelPriv::Layer &ly = mp->layers[l];
        KTRY(ctx, KID_F_RMSNORM, vk::launch_rmsnorm_rows(st, fs->h, ly.attn_norm, fs->xn, S, D, mp->eps));
        KTRY(ctx, KID_F_GEMM, vk::launch_gemm(st, vk::GEMM_PLAIN, fs->xn, ly.wqkv, fs->qkv, S, 3 * D, D, 3 * D, 0, cu));
        KTRY(ctx, KID_F_ROPE_KV,
             vk::launch_rope_kv(st, fs->qkv, fs->q, ly.kc, ly.vc, fs->freqs, offset, S, D, hd, mp->ctx));
        KTRY(ctx, KID_F_ATTN_PREFILL,
             vk::launch_attn_prefill(st, fs->q, ly.kc, ly.vc, fs->attn, offset, S, mp->H, hd, mp->ctx, scale));
        KTRY(ctx, KID_F_GEMM, vk::launch_gemm(st, vk::GEMM_RESID, fs->attn, ly.wo, fs->h, S, D, D, D, 0, cu));
        KTRY(ctx, KID_F_RMSNORM, vk::launch_rmsnorm_rows(st, fs->h, ly.ffn_norm, fs->xn, S, D, mp->eps));
        KTRY(ctx, KID_F_GEMM,
             vk::launch_gemm(st, vk::GEMM_SILU_HI, fs->xn, ly.wug, fs->ug, S, 2 * F, D, 2 * F, F, cu));
        KTRY(ctx, KID_F_SWIGLU, vk::launch_swiglu(st, fs->ug, fs->act, S, F));
        KTRY(ctx, KID_F_GEMM, vk::launch_gemm(st, vk::GEMM_RESID, fs->act, ly.wd, fs->h, S, D, F, D, 0, cu));
    }
    KTRY(ctx, KID_F_RMSNORM, vk::launch_rmsnorm_rows(st, fs->h, mp->out_norm, fs->xn, S, D, mp->eps));
    KTRY(ctx, KID_F_GEMM, vk::launch_gemm(st, vk::GEMM_PLAIN, fs->xn, mp->out_w, fs->logits, S, V, D, V, 0, cu));
    KTRY(ctx, KID_F_ARGMAX, vk::launch_argmax_rows(st, fs->logits, fs->ids, S, V));
    return VKLLM_ERR_OK;
}

vkllm_err_t fused_plan_init(vkllm_context *ctx, vkllm_graph *graph)
{
    auto *p = (FusedPlan *)graph->plan;
    ModelPriv *mp = model_priv(p->model);
    _CHECK_ARGS(mp && mp->fused_ok);
    _CHECK_ARGS(p->offset + p->S <= mp->ctx);
    _CHECK_ARGS(p->input_toks->dtype == vkllm_dtype_uint32 && p->input_toks->data.mapped);
    // decode attention keeps a whole row of scores in LDS next to an 8 KB reduction buffer
    if (p->S == 1 && (size_t)mp->ctx * sizeof(float) > 54 * 1024)
    {
        log_error("fused decode supports context_length <= %u", (unsigned)(54 * 1024 / sizeof(float)));
        return VKLLM_ERR_ARGS;
    }
    if (p->S > 1 && (size_t)(p->offset + p->S) * sizeof(float) > 60 * 1024)
    {
        log_error("prefill attention holds %u scores per row in LDS; at most %u", p->offset + p->S,
                  (unsigned)(60 * 1024 / sizeof(float)));
        return VKLLM_ERR_ARGS;
    }
    return ensure_state(ctx, mp, p->S);
}

vkllm_err_t fused_plan_run(vkllm_context *ctx, vkllm_graph *graph)
{
    auto *p = (FusedPlan *)graph->plan;
    ModelPriv *mp = model_priv(p->model);
    _CHECK(fused_plan_init(ctx, graph));
    FusedState *fs = mp->fs;
    hipStream_t st = ctx->device->stream;
    const uint32_t S = p->S;
    // step inputs: ids from the mapped input tensor's host mirror (written by vkllm_commands_upload)
    fs->step_h->offset = p->offset;
    fs->step_h->S = S;
    memcpy(fs->io_h, p->input_toks->data.host, (size_t)S * 4);
    HIP_TRY(hipMemcpyAsync(fs->step, fs->step_h, sizeof(vk::Step), hipMemcpyHostToDevice, st));
    HIP_TRY(hipMemcpyAsync(fs->toks, fs->io_h, (size_t)S * 4, hipMemcpyHostToDevice, st));
    if (S == 1)
    {
        if (ctx->device->graph_replay && !ctx->device->timing)
        {
            if (!fs->exec)
            {
                HIP_TRY(hipStreamBeginCapture(st, hipStreamCaptureModeRelaxed));
                vkllm_err_t rc = enqueue_decode(ctx, mp);
                hipGraph_t g = nullptr;
                hipError_t ce = hipStreamEndCapture(st, &g);
                if (rc != VKLLM_ERR_OK)
                {
                    if (g)
                        (void)hipGraphDestroy(g);
                    return rc;
                }
                HIP_TRY(ce);
                fs->graph = g;
                HIP_TRY(hipGraphInstantiate(&fs->exec, g, nullptr, nullptr, 0));
            }
            HIP_TRY(hipGraphLaunch(fs->exec, st));
        }
        else
            _CHECK(enqueue_decode(ctx, mp));
    }
    else
        _CHECK(enqueue_prefill(ctx, mp, S, p->offset));
    // results: arg-max ids into the output node's device memory and host mirror
    vkllm_tensor *out = graph->output_node;
    void *out_dev = tensor_dev(ctx, out);
    if (!out_dev)
        return VKLLM_ERR_ALLOC;
    HIP_TRY(hipMemcpyAsync(out_dev, fs->ids, (size_t)S * 4, hipMemcpyDeviceToDevice, st));
    HIP_TRY(hipMemcpyAsync(fs->io_h, fs->ids, (size_t)S * 4, hipMemcpyDeviceToHost, st));
    HIP_TRY(hipStreamSynchronize(st));
    out->data.valid = true;
    if (out->data.host)
        memcpy(out->data.host, fs->io_h, (size_t)S * 4);
    return VKLLM_ERR_OK;
}

// ---- extension: fused-step internals for tests and measurement ----

// Copies the fp16 logits of the last fused step ([S, vocab]) into `dst`.
extern "C" vkllm_err_t vkllm_hip_model_last_logits(struct vkllm_context *ctx, struct vkllm_models_llama2 *model,
                                                   uint16_t *dst, uint32_t rows)
{
    _CHECK_ARGS(ctx && model && dst);
    ModelPriv *mp = model_priv(model);
    _CHECK_ARGS(mp && mp->fs && mp->fs->logits && rows <= mp->fs->cap_S);
    HIP_TRY(hipMemcpyAsync(dst, mp->fs->logits, (size_t)rows * mp->V * 2, hipMemcpyDeviceToHost,
                           ctx->device->stream));
    HIP_TRY(hipStreamSynchronize(ctx->device->stream));
    return VKLLM_ERR_OK;
}

extern "C" vkllm_err_t vkllm_hip_model_time_kernel(struct vkllm_context *ctx, struct vkllm_models_llama2 *model,
                                                   const char *family, uint32_t reps, uint64_t *total_ns)
{
    _CHECK_ARGS(ctx && model && family && reps > 0 && total_ns);
    ModelPriv *mp = model_priv(model);
    _CHECK_ARGS(mp && mp->fs && mp->fs->cap_S >= 1 && mp->fs->h);
    _CHECK_ARGS(strcmp(family, "fused_gateup") == 0);
    hipStream_t st = ctx->device->stream;
    const int cu = ctx->device->cu_count;
    // one untimed launch so the first timed one does not pay for code loading
    HIP_TRY(vk::launch_gemv(st, vk::EPI_GATEUP, gateup_args(mp, 0), cu));
    hipEvent_t ev[2];
    HIP_TRY(hipEventCreate(&ev[0]));
    if (hipEventCreate(&ev[1]) != hipSuccess)
    {
        (void)hipEventDestroy(ev[0]);
        return VKLLM_ERR_VULKAN;
    }
    hipError_t e = hipEventRecord(ev[0], st);
    for (uint32_t r = 0; r < reps && e == hipSuccess; ++r)
        e = vk::launch_gemv(st, vk::EPI_GATEUP, gateup_args(mp, (r + 1) % mp->L), cu);
    if (e == hipSuccess)
        e = hipEventRecord(ev[1], st);
    if (e == hipSuccess)
        e = hipEventSynchronize(ev[1]);
    float ms = 0.f;
    if (e == hipSuccess)
        e = hipEventElapsedTime(&ms, ev[0], ev[1]);
    (void)hipEventDestroy(ev[0]);
    (void)hipEventDestroy(ev[1]);
    if (e != hipSuccess)
        return hip_fail(e, "vkllm_hip_model_time_kernel", __FILE__, __LINE__);
    *total_ns = (uint64_t)((double)ms * 1e6);
    return VKLLM_ERR_OK;
}
