// Host side of the VKLLM_OP_* operators: argument validation with the reference's error codes, kernel choice,
// and the launch on the context stream. Replaces src/core/vkllm_op_{copy,bin,embedding,rmsnorm,matmul,rope,
// softmax,ffn_up_and_gate,update_rows,arg_max}.c.
#include <cmath>
#include <cstring>

#include "runtime.h"
#include "vkllm/vkllm_op_arg_max.h"
#include "vkllm/vkllm_op_bin.h"
#include "vkllm/vkllm_op_copy.h"
#include "vkllm/vkllm_op_embedding.h"
#include "vkllm/vkllm_op_ffn_up_and_gate.h"
#include "vkllm/vkllm_op_matmul.h"
#include "vkllm/vkllm_op_rmsnorm.h"
#include "vkllm/vkllm_op_rope.h"
#include "vkllm/vkllm_op_softmax.h"
#include "vkllm/vkllm_op_update_rows.h"

static bool same_shape(const vkllm_tensor *a, const vkllm_tensor *b)
{
    return a->shapes[0] == b->shapes[0] && a->shapes[1] == b->shapes[1] && a->shapes[2] == b->shapes[2] &&
           a->shapes[3] == b->shapes[3];
}

static bool is_float(vkllm_dtype_t d)
{
    return d == vkllm_dtype_float16 || d == vkllm_dtype_float32;
}

// Every view a kernel is given must stay inside its base allocation.
static bool view_in_bounds(const vkllm_tensor *t)
{
    const vkllm_tensor *b = t;
    while (b->data.is_ref && b->srcs[0])
        b = b->srcs[0];
    uint64_t last = 0;
    for (int i = 0; i < 4; ++i)
        last += (uint64_t)(t->shapes[i] - 1) * t->strides[i];
    return last + dtype_bytes(t->dtype) <= b->bytes;
}

#define CHECK_VIEW(_t)                                                                                              \
    do                                                                                                              \
    {                                                                                                               \
        if (!view_in_bounds(_t))                                                                                    \
        {                                                                                                           \
            log_error("tensor %s: view exceeds its allocation", (_t)->name);                                        \
            return VKLLM_ERR_ARGS;                                                                                  \
        }                                                                                                           \
    } while (0)

#define LAUNCH(_ctx, _kid, _call)                                                                                   \
    do                                                                                                              \
    {                                                                                                               \
        hipError_t _e = timed((_ctx), pipeline_of((_ctx), (_kid)), [&]() { return (_call); });                     \
        if (_e != hipSuccess)                                                                                       \
            return hip_fail(_e, #_call, __FILE__, __LINE__);                                                        \
    } while (0)

#define NEED_DEV(_v)                                                                                                \
    do                                                                                                              \
    {                                                                                                               \
        if (!(_v).p)                                                                                                \
            return VKLLM_ERR_ALLOC;                                                                                 \
    } while (0)

// =============================================================================================================
// COPY: src/core/vkllm_op_copy.c:11-30 (init), :32-122 (run)
extern "C" vkllm_err_t vkllm_op_copy_init(struct vkllm_context *context, struct vkllm_commands *commands,
                                          struct vkllm_tensor *tensor)
{
    DeviceScope device_scope(context);
    _CHECK_ARGS(context && commands && tensor);
    _CHECK_ARGS(tensor->srcs[0]);
    _CHECK_ARGS(tensor->op == VKLLM_OP_COPY);
    _CHECK_ARGS(same_shape(tensor->srcs[0], tensor));
    if (tensor->dtype != tensor->srcs[0]->dtype || !is_float(tensor->dtype))
    {
        log_error("copy: unsupported dtypes %s -> %s", vkllm_dtype_s(tensor->srcs[0]->dtype),
                  vkllm_dtype_s(tensor->dtype));
        return VKLLM_ERR_ARGS;
    }
    tensor->pipeline = pipeline_of(context, KID_COPY);
    return VKLLM_ERR_OK;
}

extern "C" vkllm_err_t vkllm_op_copy_run(struct vkllm_context *context, struct vkllm_commands *commands,
                                         struct vkllm_tensor *tensor)
{
    DeviceScope device_scope(context);
    _CHECK(vkllm_op_copy_init(context, commands, tensor));
    CHECK_VIEW(tensor->srcs[0]);
    CHECK_VIEW(tensor);
    vk::TView in = tview(context, tensor->srcs[0]), out = tview(context, tensor);
    NEED_DEV(in);
    NEED_DEV(out);
    LAUNCH(context, KID_COPY, vk::launch_copy(context->device->stream, in, out));
    commands_note_write(commands, tensor);
    return VKLLM_ERR_OK;
}

extern "C" vkllm_err_t vkllm_op_copy_post_run(struct vkllm_context *, struct vkllm_commands *, struct vkllm_tensor *)
{
    return VKLLM_ERR_OK;
}

// =============================================================================================================
// BIN: src/core/vkllm_op_bin.c:9-123
extern "C" vkllm_err_t vkllm_op_bin_init(struct vkllm_context *context, struct vkllm_commands *commands,
                                         struct vkllm_tensor *tensor)
{
    DeviceScope device_scope(context);
    _CHECK_ARGS(context && commands && tensor);
    _CHECK_ARGS(tensor->srcs[0] && tensor->srcs[1]);
    _CHECK_ARGS(tensor->op == VKLLM_OP_BIN);
    vkllm_tensor *a = tensor->srcs[0], *b = tensor->srcs[1];
    _CHECK_ARGS(same_shape(a, tensor) && same_shape(b, tensor));
    int32_t op;
    memcpy(&op, tensor->params, sizeof(op));
    _CHECK_ARGS(op >= 0 && op <= 3);
    if (!is_float(tensor->dtype))
        return VKLLM_ERR_ARGS;
    if (!((a->dtype == vkllm_dtype_float16 && b->dtype == vkllm_dtype_float16) ||
          (a->dtype == vkllm_dtype_float32 && b->dtype == vkllm_dtype_float32)))
        return VKLLM_ERR_ARGS;
    tensor->pipeline = pipeline_of(context, KID_BIN);
    return VKLLM_ERR_OK;
}

extern "C" vkllm_err_t vkllm_op_bin_run(struct vkllm_context *context, struct vkllm_commands *commands,
                                        struct vkllm_tensor *tensor)
{
    DeviceScope device_scope(context);
    _CHECK(vkllm_op_bin_init(context, commands, tensor));
    CHECK_VIEW(tensor->srcs[0]);
    CHECK_VIEW(tensor->srcs[1]);
    CHECK_VIEW(tensor);
    int32_t op;
    memcpy(&op, tensor->params, sizeof(op));
    vk::TView a = tview(context, tensor->srcs[0]), b = tview(context, tensor->srcs[1]), out = tview(context, tensor);
    NEED_DEV(a);
    NEED_DEV(b);
    NEED_DEV(out);
    LAUNCH(context, KID_BIN, vk::launch_bin(context->device->stream, a, b, out, op));
    commands_note_write(commands, tensor);
    return VKLLM_ERR_OK;
}

extern "C" vkllm_err_t vkllm_op_bin_post_run(struct vkllm_context *, struct vkllm_commands *, struct vkllm_tensor *)
{
    return VKLLM_ERR_OK;
}

// =============================================================================================================
// EMBEDDING: src/core/vkllm_op_embedding.c:10-110
extern "C" vkllm_err_t vkllm_op_embedding_init(struct vkllm_context *context, struct vkllm_commands *commands,
                                               struct vkllm_tensor *tensor)
{
    DeviceScope device_scope(context);
    _CHECK_ARGS(context && commands && tensor);
    _CHECK_ARGS(tensor->srcs[0] && tensor->srcs[1]);
    vkllm_tensor *idx = tensor->srcs[0], *table = tensor->srcs[1];
    _CHECK_ARGS(idx->dtype == vkllm_dtype_uint32);
    _CHECK_ARGS(table->dtype == vkllm_dtype_float16 || table->dtype == vkllm_dtype_float32);
    _CHECK_ARGS(idx->shapes[0] == 1 && table->shapes[0] == 1 && table->shapes[1] == 1);
    if (!is_float(tensor->dtype))
        return VKLLM_ERR_ARGS;
    if (tensor->dtype != table->dtype)
        return VKLLM_ERR_PIPELINE_NOT_FOUND;
    // index (0, c, h, w) writes output row (c, h, w) (src/shaders/vkllm_embedding.comp:63); keep it in bounds
    _CHECK_ARGS(tensor->shapes[0] >= idx->shapes[1] && tensor->shapes[1] >= idx->shapes[2] &&
                tensor->shapes[2] >= idx->shapes[3] && tensor->shapes[3] >= table->shapes[3]);
    tensor->pipeline = pipeline_of(context, KID_EMBEDDING);
    return VKLLM_ERR_OK;
}

extern "C" vkllm_err_t vkllm_op_embedding_run(struct vkllm_context *context, struct vkllm_commands *commands,
                                              struct vkllm_tensor *tensor)
{
    DeviceScope device_scope(context);
    _CHECK(vkllm_op_embedding_init(context, commands, tensor));
    CHECK_VIEW(tensor->srcs[0]);
    CHECK_VIEW(tensor->srcs[1]);
    CHECK_VIEW(tensor);
    uint32_t unk;
    memcpy(&unk, tensor->params, sizeof(unk));
    vk::TView idx = tview(context, tensor->srcs[0]), table = tview(context, tensor->srcs[1]),
              out = tview(context, tensor);
    NEED_DEV(idx);
    NEED_DEV(table);
    NEED_DEV(out);
    LAUNCH(context, KID_EMBEDDING, vk::launch_embedding(context->device->stream, idx, table, out, unk));
    commands_note_write(commands, tensor);
    return VKLLM_ERR_OK;
}

extern "C" vkllm_err_t vkllm_op_embedding_post_run(struct vkllm_context *, struct vkllm_commands *,
                                                   struct vkllm_tensor *)
{
    return VKLLM_ERR_OK;
}

// =============================================================================================================
// RMSNORM: src/core/vkllm_op_rmsnorm.c:11-124 (only fp16 in / fp32 weight / fp16 out has a kernel)
extern "C" vkllm_err_t vkllm_op_rmsnorm_init(struct vkllm_context *context, struct vkllm_commands *commands,
                                             struct vkllm_tensor *tensor)
{
    DeviceScope device_scope(context);
    _CHECK_ARGS(context && commands && tensor);
    _CHECK_ARGS(tensor->srcs[0] && tensor->srcs[1]);
    _CHECK_ARGS(tensor->op == VKLLM_OP_RMSNORM);
    vkllm_tensor *x = tensor->srcs[0], *w = tensor->srcs[1];
    _CHECK_ARGS(same_shape(x, tensor));
    _CHECK_ARGS(w->shapes[0] == 1 && w->shapes[1] == 1 && w->shapes[2] == 1);
    _CHECK_ARGS(w->shapes[3] == x->shapes[3]);
    if (!(tensor->dtype == vkllm_dtype_float16 && x->dtype == vkllm_dtype_float16 && w->dtype == vkllm_dtype_float32))
        return VKLLM_ERR_PIPELINE_NOT_FOUND;
    tensor->pipeline = pipeline_of(context, KID_RMSNORM);
    return VKLLM_ERR_OK;
}

extern "C" vkllm_err_t vkllm_op_rmsnorm_run(struct vkllm_context *context, struct vkllm_commands *commands,
                                            struct vkllm_tensor *tensor)
{
    DeviceScope device_scope(context);
    _CHECK(vkllm_op_rmsnorm_init(context, commands, tensor));
    CHECK_VIEW(tensor->srcs[0]);
    CHECK_VIEW(tensor->srcs[1]);
    CHECK_VIEW(tensor);
    vkllm_op_rmsnorm_params p;
    memcpy(&p, tensor->params, sizeof(p));
    vk::TView x = tview(context, tensor->srcs[0]), w = tview(context, tensor->srcs[1]), out = tview(context, tensor);
    NEED_DEV(x);
    NEED_DEV(w);
    NEED_DEV(out);
    // contiguous rows of a multiple of 8 take the fused step's row kernel (512 threads, 16-byte vectors)
    const uint32_t D = x.n[3];
    const uint64_t rows = (uint64_t)x.n[0] * x.n[1] * x.n[2];
    auto packed = [D](const vk::TView &v) {
        return v.s[3] == 1 && v.s[2] == D && v.s[1] == v.n[2] * D && v.s[0] == v.n[1] * v.s[1] &&
               (uintptr_t)v.p % 16 == 0;
    };
    if (D % 8 == 0 && rows <= 0x7fffffffu && packed(x) && packed(out) && w.s[3] == 1 && (uintptr_t)w.p % 16 == 0)
        LAUNCH(context, KID_RMSNORM,
               vk::launch_rmsnorm_rows(context->device->stream, (const uint16_t *)x.p, (const float *)w.p,
                                       (uint16_t *)out.p, (uint32_t)rows, D, p.eps, false));
    else
        LAUNCH(context, KID_RMSNORM, vk::launch_rmsnorm(context->device->stream, x, w, out, p.eps));
    commands_note_write(commands, tensor);
    return VKLLM_ERR_OK;
}

extern "C" vkllm_err_t vkllm_op_rmsnorm_post_run(struct vkllm_context *, struct vkllm_commands *,
                                                 struct vkllm_tensor *)
{
    return VKLLM_ERR_OK;
}

// =============================================================================================================
// MATMUL: src/core/vkllm_op_matmul.c:14-339

// src/core/vkllm_op_matmul.c:14-24
static bool is_transposed_b(const vkllm_tensor *t)
{
    const vkllm_tensor *a = t->srcs[0], *b = t->srcs[1];
    uint32_t M = t->shapes[2], N = t->shapes[3], K = a->shapes[3];
    return a->shapes[2] == M && b->shapes[2] == N && a->shapes[3] == K && b->shapes[3] == K;
}

// src/core/vkllm_op_matmul.c:26-30
static bool is_mat_mul_vec(const vkllm_tensor *t)
{
    return t->srcs[0]->shapes[2] == 1 && is_transposed_b(t);
}

// The matrix-core and streaming kernels of the fused token step serve the op when its operands have their layout:
// fp16 A [1,1,M,K], B [1,1,N,K] (is_transposed_b) and out [1,1,M,N], rows contiguous, K a multiple of 8, 16-byte
// aligned rows, scale 1. M == 1 (the reference's mat_mul_vec case) takes the streaming GEMV (16-byte weight loads,
// fp32 accumulation, DPP wave sums) when act is 0; M > 1 takes the MFMA tile GEMM, act 1 as its SiLU epilogue.
// Anything else (fp32, broadcast batches, B as [K, N], a scale, strided views) runs the generic kernels. Both keep
// the reference's rounding points (fp32 sums, then fp16(act(scale * acc))), so only the fp32 summation order differs.
enum MatmulPath
{
    GENERIC,
    FAST_GEMV,
    FAST_GEMM
};

static bool rows_fp16(const vk::TView &v, uint32_t rows, uint32_t cols)
{
    return v.dt == vkllm_dtype_float16 && v.n[0] == 1 && v.n[1] == 1 && v.n[2] == rows && v.n[3] == cols &&
           v.s[3] == 1 && (rows == 1 || v.s[2] % 8 == 0) && (uintptr_t)v.p % 16 == 0;
}

static MatmulPath matmul_fast_path(const vk::TView &a, const vk::TView &b, const vk::TView &out,
                                   const vkllm_op_matmul_params &p, bool transposed_b)
{
    const uint32_t M = out.n[2], N = out.n[3], K = a.n[3];
    if (!transposed_b || p.scale != 1.0f || K % 8 != 0 || !rows_fp16(a, M, K) || !rows_fp16(b, N, K) ||
        !rows_fp16(out, M, N) || (M > 1 && a.s[2] != K) || b.s[2] != K)
        return GENERIC;
    if (M == 1)
        return p.act == 0 ? FAST_GEMV : GENERIC;
    return p.act == 0 || p.act == 1 ? FAST_GEMM : GENERIC;
}

static hipError_t launch_op_gemv(vkllm_context *ctx, const vk::TView &a, const vk::TView &b, const vk::TView &out)
{
    vk::GemvArgs g{};
    g.x = (const uint16_t *)a.p;
    g.w = (const uint16_t *)b.p;
    g.K = a.n[3];
    g.rows = out.n[3];
    g.units = (g.rows + 1) / 2;
    g.out = (uint16_t *)out.p;
    return vk::launch_gemv(ctx->device->stream, vk::EPI_RAW, g, ctx->device->cu_count);
}

// 64 MB of split-K partials for the op's tile GEMM, made once per context (the kernels then split K only as far as
// it fits); an allocation failure leaves K unsplit
static vkllm_err_t op_gemm_workspace(vkllm_context *ctx, float **work, size_t *elems)
{
    vkllm_gpu_device *dev = ctx->device;
    if (!dev->op_work)
    {
        const size_t want = (size_t)16 << 20;
        if (hipMalloc(&dev->op_work, want * sizeof(float)) == hipSuccess)
            dev->op_work_elems = want;
        else
        {
            (void)hipGetLastError();
            dev->op_work = nullptr;
            dev->op_work_elems = 0;
        }
    }
    *work = dev->op_work;
    *elems = dev->op_work_elems;
    return VKLLM_ERR_OK;
}

extern "C" vkllm_err_t vkllm_op_matmul_init(struct vkllm_context *context, struct vkllm_commands *commands,
                                            struct vkllm_tensor *tensor)
{
    DeviceScope device_scope(context);
    _CHECK_ARGS(context && commands && tensor);
    _CHECK_ARGS(tensor->srcs[0] && tensor->srcs[1]);
    _CHECK_ARGS(tensor->op == VKLLM_OP_MATMUL);
    vkllm_tensor *a = tensor->srcs[0], *b = tensor->srcs[1];
    if (a->dtype == vkllm_dtype_float16 && b->dtype == vkllm_dtype_float16)
    {
        if (tensor->dtype != vkllm_dtype_float16)
        {
            log_error("input dtype = fp16 and output dtype != fp16");
            return VKLLM_ERR_PIPELINE_NOT_FOUND;
        }
    }
    else if (!(a->dtype == vkllm_dtype_float32 && b->dtype == vkllm_dtype_float32 &&
               tensor->dtype == vkllm_dtype_float32))
        return VKLLM_ERR_PIPELINE_NOT_FOUND;
    tensor->pipeline = pipeline_of(context, is_mat_mul_vec(tensor) ? KID_GEMV : KID_GEMM);
    return VKLLM_ERR_OK;
}

extern "C" vkllm_err_t vkllm_op_matmul_run(struct vkllm_context *context, struct vkllm_commands *commands,
                                           struct vkllm_tensor *tensor)
{
    DeviceScope device_scope(context);
    _CHECK(vkllm_op_matmul_init(context, commands, tensor));
    vkllm_tensor *a = tensor->srcs[0], *b = tensor->srcs[1];
    const uint32_t M = tensor->shapes[2], N = tensor->shapes[3], K = a->shapes[3];
    const bool tb = is_transposed_b(tensor);
    _CHECK_ARGS(a->shapes[2] == M); // src/core/vkllm_op_matmul.c:234
    if (!tb)
        _CHECK_ARGS(b->shapes[3] == N && b->shapes[2] == K); // src/core/vkllm_op_matmul.c:238-241
    for (int d = 0; d < 2; ++d)
    {
        _CHECK_ARGS(a->shapes[d] == 1 || a->shapes[d] == tensor->shapes[d]);
        _CHECK_ARGS(b->shapes[d] == 1 || b->shapes[d] == tensor->shapes[d]);
    }
    CHECK_VIEW(a);
    CHECK_VIEW(b);
    CHECK_VIEW(tensor);
    vkllm_op_matmul_params p;
    memcpy(&p, tensor->params, sizeof(p));
    vk::TView av = tview(context, a), bv = tview(context, b), out = tview(context, tensor);
    NEED_DEV(av);
    NEED_DEV(bv);
    NEED_DEV(out);
    const KernelId kid = is_mat_mul_vec(tensor) ? KID_GEMV : KID_GEMM;
    switch (matmul_fast_path(av, bv, out, p, tb))
    {
    case FAST_GEMV:
        LAUNCH(context, kid, launch_op_gemv(context, av, bv, out));
        break;
    case FAST_GEMM:
    {
        float *work = nullptr;
        size_t work_elems = 0;
        _CHECK(op_gemm_workspace(context, &work, &work_elems));
        LAUNCH(context, kid,
               vk::launch_gemm(context->device->stream, p.act ? vk::GEMM_SILU_HI : vk::GEMM_PLAIN,
                               (const uint16_t *)av.p, (const uint16_t *)bv.p, (uint16_t *)out.p, M, N, K, out.s[2], 0,
                               context->device->cu_count, work, work_elems));
        break;
    }
    default:
        LAUNCH(context, kid, vk::launch_matmul(context->device->stream, av, bv, out, p.scale, p.act, tb));
    }
    commands_note_write(commands, tensor);
    return VKLLM_ERR_OK;
}

extern "C" vkllm_err_t vkllm_op_matmul_post_run(struct vkllm_context *, struct vkllm_commands *,
                                                struct vkllm_tensor *)
{
    return VKLLM_ERR_OK;
}

// =============================================================================================================
// ROPE: src/core/vkllm_op_rope.c:8-153
extern "C" vkllm_err_t vkllm_op_rope_init(struct vkllm_context *context, struct vkllm_commands *commands,
                                          struct vkllm_tensor *tensor)
{
    DeviceScope device_scope(context);
    _CHECK_ARGS(context && commands && tensor);
    _CHECK_ARGS(tensor->srcs[0]);
    _CHECK_ARGS(tensor->op == VKLLM_OP_ROPE);
    vkllm_tensor *in = tensor->srcs[0];
    _CHECK_ARGS(same_shape(in, tensor));
    if (!is_float(in->dtype))
    {
        log_error("unsupported op input dtype: %s", vkllm_dtype_s(in->dtype));
        return VKLLM_ERR_ARGS;
    }
    _CHECK_ARGS(in->dtype == tensor->dtype);
    _CHECK_ARGS(in->shapes[3] % 2 == 0 && in->shapes[3] / 2 <= (uint32_t)vk::kMaxRopeFreqs);
    tensor->pipeline = pipeline_of(context, KID_ROPE);
    return VKLLM_ERR_OK;
}

extern "C" vkllm_err_t vkllm_op_rope_run(struct vkllm_context *context, struct vkllm_commands *commands,
                                         struct vkllm_tensor *tensor)
{
    DeviceScope device_scope(context);
    _CHECK(vkllm_op_rope_init(context, commands, tensor));
    CHECK_VIEW(tensor->srcs[0]);
    CHECK_VIEW(tensor);
    vkllm_op_rope_params p;
    memcpy(&p, tensor->params, sizeof(p));
    const uint32_t D = tensor->srcs[0]->shapes[3];
    float freqs[vk::kMaxRopeFreqs];
    for (uint32_t w = 0; w < D / 2; ++w)
        freqs[w] = powf(p.base, (float)(2 * w) / (float)D); // base^(2w/D), src/shaders/vkllm_rope.comp:68
    vk::TView in = tview(context, tensor->srcs[0]), out = tview(context, tensor);
    NEED_DEV(in);
    NEED_DEV(out);
    LAUNCH(context, KID_ROPE, vk::launch_rope(context->device->stream, in, out, p.offset, freqs, p.neox_style));
    commands_note_write(commands, tensor);
    return VKLLM_ERR_OK;
}

extern "C" vkllm_err_t vkllm_op_rope_post_run(struct vkllm_context *, struct vkllm_commands *, struct vkllm_tensor *)
{
    return VKLLM_ERR_OK;
}

// =============================================================================================================
// SOFTMAX: src/core/vkllm_op_softmax.c:8-115
extern "C" vkllm_err_t vkllm_op_softmax_init(struct vkllm_context *context, struct vkllm_commands *commands,
                                             struct vkllm_tensor *tensor)
{
    DeviceScope device_scope(context);
    _CHECK_ARGS(context && commands && tensor);
    _CHECK_ARGS(tensor->srcs[0]);
    _CHECK_ARGS(tensor->op == VKLLM_OP_SOFTMAX);
    vkllm_tensor *in = tensor->srcs[0];
    _CHECK_ARGS(same_shape(in, tensor));
    if (tensor->dtype != in->dtype)
    {
        log_error("softmax input and output dtype mismatch: input=%s, output=%s", vkllm_dtype_s(in->dtype),
                  vkllm_dtype_s(tensor->dtype));
        return VKLLM_ERR_ARGS;
    }
    if (!is_float(in->dtype))
        return VKLLM_ERR_ARGS;
    tensor->pipeline = pipeline_of(context, KID_SOFTMAX);
    return VKLLM_ERR_OK;
}

extern "C" vkllm_err_t vkllm_op_softmax_run(struct vkllm_context *context, struct vkllm_commands *commands,
                                            struct vkllm_tensor *tensor)
{
    DeviceScope device_scope(context);
    _CHECK(vkllm_op_softmax_init(context, commands, tensor));
    CHECK_VIEW(tensor->srcs[0]);
    CHECK_VIEW(tensor);
    vkllm_op_softmax_params p;
    memcpy(&p, tensor->params, sizeof(p));
    vk::TView in = tview(context, tensor->srcs[0]), out = tview(context, tensor);
    NEED_DEV(in);
    NEED_DEV(out);
    LAUNCH(context, KID_SOFTMAX, vk::launch_softmax(context->device->stream, in, out, p.seq_mask, p.offsets));
    commands_note_write(commands, tensor);
    return VKLLM_ERR_OK;
}

extern "C" vkllm_err_t vkllm_op_softmax_post_run(struct vkllm_context *, struct vkllm_commands *,
                                                 struct vkllm_tensor *)
{
    return VKLLM_ERR_OK;
}

// =============================================================================================================
// UPDATE_ROWS: src/core/vkllm_op_update_rows.c:8-104
extern "C" vkllm_err_t vkllm_op_update_rows_init(struct vkllm_context *context, struct vkllm_commands *commands,
                                                 struct vkllm_tensor *tensor)
{
    DeviceScope device_scope(context);
    _CHECK_ARGS(context && commands && tensor);
    _CHECK_ARGS(tensor->srcs[0]);
    _CHECK_ARGS(tensor->op == VKLLM_OP_UPDATE_ROWS);
    vkllm_tensor *in = tensor->srcs[0];
    _CHECK_ARGS(in->shapes[0] == tensor->shapes[0]);
    _CHECK_ARGS(in->shapes[1] == tensor->shapes[1]);
    _CHECK_ARGS(in->shapes[3] == tensor->shapes[3]);
    vkllm_op_update_rows_params p;
    memcpy(&p, tensor->params, sizeof(p));
    _CHECK_ARGS(p.offset_rows + in->shapes[2] <= tensor->shapes[2]);
    if (tensor->dtype != in->dtype)
    {
        log_error("update_rows input and output dtype mismatch: input=%s, output=%s", vkllm_dtype_s(in->dtype),
                  vkllm_dtype_s(tensor->dtype));
        return VKLLM_ERR_ARGS;
    }
    if (!is_float(in->dtype))
        return VKLLM_ERR_ARGS;
    tensor->pipeline = pipeline_of(context, KID_UPDATE_ROWS);
    return VKLLM_ERR_OK;
}

extern "C" vkllm_err_t vkllm_op_update_rows_run(struct vkllm_context *context, struct vkllm_commands *commands,
                                                struct vkllm_tensor *tensor)
{
    DeviceScope device_scope(context);
    _CHECK(vkllm_op_update_rows_init(context, commands, tensor));
    CHECK_VIEW(tensor->srcs[0]);
    CHECK_VIEW(tensor);
    vkllm_op_update_rows_params p;
    memcpy(&p, tensor->params, sizeof(p));
    vk::TView in = tview(context, tensor->srcs[0]), out = tview(context, tensor);
    NEED_DEV(in);
    NEED_DEV(out);
    LAUNCH(context, KID_UPDATE_ROWS, vk::launch_update_rows(context->device->stream, in, out, p.offset_rows));
    commands_note_write(commands, tensor);
    return VKLLM_ERR_OK;
}

extern "C" vkllm_err_t vkllm_op_update_rows_post_run(struct vkllm_context *, struct vkllm_commands *,
                                                     struct vkllm_tensor *)
{
    return VKLLM_ERR_OK;
}

// =============================================================================================================
// ARG_MAX: src/core/vkllm_op_arg_max.c:9-121
extern "C" vkllm_err_t vkllm_op_arg_max_init(struct vkllm_context *context, struct vkllm_commands *commands,
                                             struct vkllm_tensor *tensor)
{
    DeviceScope device_scope(context);
    _CHECK_ARGS(context && commands && tensor);
    _CHECK_ARGS(tensor->srcs[0]);
    _CHECK_ARGS(tensor->op == VKLLM_OP_ARG_MAX);
    vkllm_tensor *in = tensor->srcs[0];
    _CHECK_ARGS(in->shapes[0] == tensor->shapes[0]);
    _CHECK_ARGS(in->shapes[1] == tensor->shapes[1]);
    _CHECK_ARGS(in->shapes[2] == tensor->shapes[2]);
    _CHECK_ARGS(tensor->shapes[3] == 1);
    if (tensor->dtype != vkllm_dtype_uint32)
    {
        log_error("arg_max output dtype must be uint32, got %s", vkllm_dtype_s(tensor->dtype));
        return VKLLM_ERR_ARGS;
    }
    if (!is_float(in->dtype))
        return VKLLM_ERR_ARGS;
    tensor->pipeline = pipeline_of(context, KID_ARG_MAX);
    return VKLLM_ERR_OK;
}

extern "C" vkllm_err_t vkllm_op_arg_max_run(struct vkllm_context *context, struct vkllm_commands *commands,
                                            struct vkllm_tensor *tensor)
{
    DeviceScope device_scope(context);
    _CHECK(vkllm_op_arg_max_init(context, commands, tensor));
    CHECK_VIEW(tensor->srcs[0]);
    CHECK_VIEW(tensor);
    vk::TView in = tview(context, tensor->srcs[0]), out = tview(context, tensor);
    NEED_DEV(in);
    NEED_DEV(out);
    LAUNCH(context, KID_ARG_MAX, vk::launch_arg_max(context->device->stream, in, out));
    commands_note_write(commands, tensor);
    return VKLLM_ERR_OK;
}

extern "C" vkllm_err_t vkllm_op_arg_max_post_run(struct vkllm_context *, struct vkllm_commands *,
                                                 struct vkllm_tensor *)
{
    return VKLLM_ERR_OK;
}

// =============================================================================================================
// FFN_UP_AND_GATE: src/core/vkllm_op_ffn_up_and_gate.c:9-164
extern "C" vkllm_err_t vkllm_op_ffn_up_and_gate_init(struct vkllm_context *context, struct vkllm_commands *commands,
                                                     struct vkllm_tensor *tensor)
{
    DeviceScope device_scope(context);
    _CHECK_ARGS(context && commands && tensor);
    _CHECK_ARGS(tensor->srcs[0] && tensor->srcs[1] && tensor->srcs[2]);
    _CHECK_ARGS(tensor->op == VKLLM_OP_FFN_UP_AND_GATE);
    vkllm_tensor *x = tensor->srcs[0], *wu = tensor->srcs[1], *wg = tensor->srcs[2];
    if (x->dtype == vkllm_dtype_float16 && wu->dtype == vkllm_dtype_float16 && wg->dtype == vkllm_dtype_float16)
    {
        if (!is_float(tensor->dtype))
            return VKLLM_ERR_PIPELINE_NOT_FOUND;
    }
    else if (!(x->dtype == vkllm_dtype_float32 && wu->dtype == vkllm_dtype_float32 &&
               wg->dtype == vkllm_dtype_float32 && tensor->dtype == vkllm_dtype_float32))
        return VKLLM_ERR_PIPELINE_NOT_FOUND;
    const uint32_t K = x->shapes[3], N = wu->shapes[2];
    _CHECK_ARGS(wu->shapes[3] == K && wg->shapes[3] == K && wg->shapes[2] == N);
    _CHECK_ARGS(wu->shapes[0] == 1 && wu->shapes[1] == 1 && wg->shapes[0] == 1 && wg->shapes[1] == 1);
    _CHECK_ARGS(tensor->shapes[0] == x->shapes[0] && tensor->shapes[1] == x->shapes[1] &&
                tensor->shapes[2] == x->shapes[2] && tensor->shapes[3] == N);
    tensor->pipeline = pipeline_of(context, KID_FFN);
    return VKLLM_ERR_OK;
}

extern "C" vkllm_err_t vkllm_op_ffn_up_and_gate_run(struct vkllm_context *context, struct vkllm_commands *commands,
                                                    struct vkllm_tensor *tensor)
{
    DeviceScope device_scope(context);
    _CHECK(vkllm_op_ffn_up_and_gate_init(context, commands, tensor));
    for (int i = 0; i < 3; ++i)
        CHECK_VIEW(tensor->srcs[i]);
    CHECK_VIEW(tensor);
    vk::TView x = tview(context, tensor->srcs[0]), wu = tview(context, tensor->srcs[1]),
              wg = tview(context, tensor->srcs[2]), out = tview(context, tensor);
    NEED_DEV(x);
    NEED_DEV(wu);
    NEED_DEV(wg);
    NEED_DEV(out);
    LAUNCH(context, KID_FFN, vk::launch_ffn_up_and_gate(context->device->stream, x, wu, wg, out));
    commands_note_write(commands, tensor);
    return VKLLM_ERR_OK;
}

extern "C" vkllm_err_t vkllm_op_ffn_up_and_gate_post_run(struct vkllm_context *, struct vkllm_commands *,
                                                         struct vkllm_tensor *)
{
    return VKLLM_ERR_OK;
}

// =============================================================================================================
// dispatch by tag (src/core/vkllm_graph.c:80-121, 162-203, 248-289)
vkllm_err_t op_init(vkllm_context *ctx, vkllm_commands *cmds, vkllm_tensor *t)
{
    switch (t->op)
    {
    case VKLLM_OP_NONE:
    case VKLLM_OP_REF:
        return VKLLM_ERR_OK;
    case VKLLM_OP_COPY:
        return vkllm_op_copy_init(ctx, cmds, t);
    case VKLLM_OP_BIN:
        return vkllm_op_bin_init(ctx, cmds, t);
    case VKLLM_OP_EMBEDDING:
        return vkllm_op_embedding_init(ctx, cmds, t);
    case VKLLM_OP_RMSNORM:
        return vkllm_op_rmsnorm_init(ctx, cmds, t);
    case VKLLM_OP_MATMUL:
        return vkllm_op_matmul_init(ctx, cmds, t);
    case VKLLM_OP_ROPE:
        return vkllm_op_rope_init(ctx, cmds, t);
    case VKLLM_OP_SOFTMAX:
        return vkllm_op_softmax_init(ctx, cmds, t);
    case VKLLM_OP_FFN_UP_AND_GATE:
        return vkllm_op_ffn_up_and_gate_init(ctx, cmds, t);
    case VKLLM_OP_UPDATE_ROWS:
        return vkllm_op_update_rows_init(ctx, cmds, t);
    case VKLLM_OP_ARG_MAX:
        return vkllm_op_arg_max_init(ctx, cmds, t);
    default:
        log_error("Unknown operation type: %d", (int)t->op);
        return VKLLM_ERR_ARGS;
    }
}

vkllm_err_t op_run(vkllm_context *ctx, vkllm_commands *cmds, vkllm_tensor *t)
{
    switch (t->op)
    {
    case VKLLM_OP_NONE:
    case VKLLM_OP_REF:
        return VKLLM_ERR_OK;
    case VKLLM_OP_COPY:
        return vkllm_op_copy_run(ctx, cmds, t);
    case VKLLM_OP_BIN:
        return vkllm_op_bin_run(ctx, cmds, t);
    case VKLLM_OP_EMBEDDING:
        return vkllm_op_embedding_run(ctx, cmds, t);
    case VKLLM_OP_RMSNORM:
        return vkllm_op_rmsnorm_run(ctx, cmds, t);
    case VKLLM_OP_MATMUL:
        return vkllm_op_matmul_run(ctx, cmds, t);
    case VKLLM_OP_ROPE:
        return vkllm_op_rope_run(ctx, cmds, t);
    case VKLLM_OP_SOFTMAX:
        return vkllm_op_softmax_run(ctx, cmds, t);
    case VKLLM_OP_FFN_UP_AND_GATE:
        return vkllm_op_ffn_up_and_gate_run(ctx, cmds, t);
    case VKLLM_OP_UPDATE_ROWS:
        return vkllm_op_update_rows_run(ctx, cmds, t);
    case VKLLM_OP_ARG_MAX:
        return vkllm_op_arg_max_run(ctx, cmds, t);
    default:
        log_error("Unknown operation type: %d", (int)t->op);
        return VKLLM_ERR_ARGS;
    }
}

vkllm_err_t op_post_run(vkllm_context *ctx, vkllm_commands *cmds, vkllm_tensor *t)
{
    (void)ctx;
    (void)cmds;
    if ((int)t->op < 0 || (int)t->op >= (int)VKLLM_OP_COUNTS)
    {
        log_error("Unknown operation type: %d", (int)t->op);
        return VKLLM_ERR_ARGS;
    }
    return VKLLM_ERR_OK;
}

// =============================================================================================================
// vkllm_hip_time_ops (vkllm_hip.h): back-to-back op launches between one hipEvent pair on the context's stream
extern "C" vkllm_err_t vkllm_hip_time_ops(struct vkllm_context *context, struct vkllm_tensor *const *tensors,
                                          uint32_t n, uint32_t reps, uint64_t *total_ns)
{
    DeviceScope device_scope(context);
    _CHECK_ARGS(context && tensors && n > 0 && reps > 0 && total_ns);
    vkllm_commands *cmds = nullptr;
    _CHECK(vkllm_commands_new(context, &cmds));
    vkllm_gpu_device *dev = context->device;
    const int timing = dev->timing;
    dev->timing = 0; // no per-launch events inside the timed region
    hipEvent_t b = nullptr, e = nullptr;
    vkllm_err_t rc = VKLLM_ERR_OK;
    // every op once first: argument checks, and first-use allocations stay outside the region
    for (uint32_t i = 0; i < n && rc == VKLLM_ERR_OK; ++i)
        rc = tensors[i] ? op_run(context, cmds, tensors[i]) : VKLLM_ERR_ARGS;
    if (rc == VKLLM_ERR_OK && (hipEventCreate(&b) != hipSuccess || hipEventCreate(&e) != hipSuccess ||
                               hipEventRecord(b, dev->stream) != hipSuccess))
        rc = VKLLM_ERR_VULKAN;
    for (uint32_t r = 0; r < reps && rc == VKLLM_ERR_OK; ++r)
        rc = op_run(context, cmds, tensors[r % n]);
    float ms = 0.f;
    if (rc == VKLLM_ERR_OK && (hipEventRecord(e, dev->stream) != hipSuccess || hipEventSynchronize(e) != hipSuccess ||
                               hipEventElapsedTime(&ms, b, e) != hipSuccess))
        rc = VKLLM_ERR_VULKAN;
    if (rc == VKLLM_ERR_OK)
        *total_ns = (uint64_t)((double)ms * 1e6);
    (void)hipStreamSynchronize(dev->stream);
    if (b)
        (void)hipEventDestroy(b);
    if (e)
        (void)hipEventDestroy(e);
    dev->timing = timing;
    vkllm_commands_free(context, cmds);
    return rc;
}
