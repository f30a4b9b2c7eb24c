// LLaMA-2 model: GGUF load into HBM weight slabs, KV cache, per-step graph construction, tokenizer.
// Replaces src/models/vkllm_models_llama2.c, src/models/vkllm_llama2_layers.c, src/models/vkllm_kvcache.c.
// The graph built here has the reference's nodes (same names, ops, shapes, params and sources, added in the same
// order); it also carries a fused plan that executes the whole step with the fused kernels.
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <unordered_set>
#include <vector>

#include "gguf.h"
#include "model_priv.h"
#include "vkllm/vkllm_graph.h"
#include "vkllm/vkllm_kvcache.h"
#include "vkllm/vkllm_llama2_layers.h"
#include "vkllm/vkllm_models_llama2.h"
#include "vkllm/vkllm_op_matmul.h"
#include "vkllm/vkllm_op_rmsnorm.h"
#include "vkllm/vkllm_op_rope.h"
#include "vkllm/vkllm_op_softmax.h"
#include "vkllm/vkllm_op_update_rows.h"

// =============================================================================================================
// KV cache: src/models/vkllm_kvcache.c:12-124

struct KvPriv
{
    std::vector<vkllm_tensor *> views;
};

extern "C" vkllm_err_t vkllm_kvcache_new(struct vkllm_context *context, uint32_t kcache_shape[4],
                                         uint32_t vcache_shape[4], uint32_t layer_counts,
                                         struct vkllm_kvcache **kvcache)
{
    DeviceScope device_scope(context);
    _CHECK_ARGS(context && kcache_shape && vcache_shape && kvcache);
    auto *p = (vkllm_kvcache *)calloc(1, sizeof(vkllm_kvcache));
    if (!p)
        return VKLLM_ERR_ALLOC;
    p->layer_counts = layer_counts;
    _ASSIGN4(p->kcache_shape, kcache_shape);
    _ASSIGN4(p->vcache_shape, vcache_shape);
    p->priv = new KvPriv();
    vkllm_err_t rc = vkllm_array_tensor_new(&p->kcaches, layer_counts);
    if (rc == VKLLM_ERR_OK)
        rc = vkllm_array_tensor_new(&p->vcaches, layer_counts);
    char name[128];
    for (uint32_t i = 0; i < layer_counts && rc == VKLLM_ERR_OK; ++i)
    {
        uint32_t offsets = 0;
        vkllm_tensor *kc = nullptr, *vc = nullptr;
        snprintf(name, sizeof(name), "kcache_%u", i);
        rc = vkllm_tensor_new(context, name, kcache_shape, vkllm_dtype_float16, VKLLM_OP_UPDATE_ROWS, nullptr, 0,
                              &offsets, sizeof(offsets), false, &kc);
        if (rc != VKLLM_ERR_OK)
            break;
        vkllm_array_tensor_append(p->kcaches, kc);
        snprintf(name, sizeof(name), "vcache_%u", i);
        rc = vkllm_tensor_new(context, name, vcache_shape, vkllm_dtype_float16, VKLLM_OP_UPDATE_ROWS, nullptr, 0,
                              &offsets, sizeof(offsets), false, &vc);
        if (rc != VKLLM_ERR_OK)
            break;
        vkllm_array_tensor_append(p->vcaches, vc);
        // caches start zeroed so every read position holds a defined value
        if (hipMemsetAsync(kc->data.dev, 0, kc->bytes, context->device->stream) != hipSuccess ||
            hipMemsetAsync(vc->data.dev, 0, vc->bytes, context->device->stream) != hipSuccess)
            rc = VKLLM_ERR_VULKAN;
        kc->data.valid = vc->data.valid = true;
    }
    if (rc != VKLLM_ERR_OK)
    {
        vkllm_kvcache_free(context, p);
        return rc;
    }
    *kvcache = p;
    return VKLLM_ERR_OK;
}

extern "C" vkllm_err_t vkllm_kvcache_update(struct vkllm_context *context, struct vkllm_kvcache *kvcache,
                                            struct vkllm_tensor **key, struct vkllm_tensor **value, uint32_t layer,
                                            uint32_t offset)
{
    DeviceScope device_scope(context);
    _CHECK_ARGS(context && kvcache && key && value);
    vkllm_tensor *pk = *key, *pv = *value;
    _CHECK_ARGS(pk && pv);
    _CHECK_ARGS(layer < kvcache->kcaches->used_n && layer < kvcache->vcaches->used_n);
    vkllm_tensor *kc = kvcache->kcaches->data[layer];
    _CHECK_ARGS(pk->shapes[0] <= kc->shapes[0]);
    _CHECK_ARGS(pk->shapes[1] <= kc->shapes[1]);
    _CHECK_ARGS(pk->shapes[2] + offset <= kc->shapes[2]);
    _CHECK_ARGS(pk->shapes[3] <= kc->shapes[3]);
    vkllm_tensor *vc = kvcache->vcaches->data[layer];
    _CHECK_ARGS(pv->shapes[0] <= vc->shapes[0]);
    _CHECK_ARGS(pv->shapes[1] <= vc->shapes[1]);
    _CHECK_ARGS(pv->shapes[2] + offset <= vc->shapes[2]);
    _CHECK_ARGS(pv->shapes[3] <= vc->shapes[3]);
    kc->srcs[0] = pk;
    memcpy(kc->params, &offset, sizeof(offset));
    vc->srcs[0] = pv;
    memcpy(vc->params, &offset, sizeof(offset));
    uint32_t extents[4] = {pk->shapes[0], pk->shapes[1], pk->shapes[2] + offset, pk->shapes[3]};
    _CHECK(vkllm_tensor_slice0(context, kc, extents, key));
    _CHECK(vkllm_tensor_slice0(context, vc, extents, value));
    auto *kp = (KvPriv *)kvcache->priv;
    kp->views.push_back(*key);
    kp->views.push_back(*value);
    return VKLLM_ERR_OK;
}

extern "C" void vkllm_kvcache_free(struct vkllm_context *context, struct vkllm_kvcache *kvcache)
{
    DeviceScope device_scope(context);
    if (!kvcache)
        return;
    if (kvcache->kcaches)
    {
        for (size_t i = 0; i < kvcache->kcaches->used_n; ++i)
            vkllm_tensor_free(context, kvcache->kcaches->data[i]);
        vkllm_array_tensor_free(kvcache->kcaches);
    }
    if (kvcache->vcaches)
    {
        for (size_t i = 0; i < kvcache->vcaches->used_n; ++i)
            vkllm_tensor_free(context, kvcache->vcaches->data[i]);
        vkllm_array_tensor_free(kvcache->vcaches);
    }
    auto *kp = (KvPriv *)kvcache->priv;
    if (kp)
    {
        for (vkllm_tensor *t : kp->views)
            vkllm_tensor_free(context, t);
        delete kp;
    }
    free(kvcache);
}

// =============================================================================================================
// load: src/models/vkllm_models_llama2.c:67-412

static void set_defaults(vkllm_models_llama2 *m) // src/models/vkllm_models_llama2.c:224-241
{
    m->meta.block_count = 32;
    m->meta.context_length = 2048;
    m->meta.embedding_length = 4096;
    m->meta.rope_freq_base = 10000.0f;
    m->meta.layer_norm_rms_epsilon = 1e-6f;
    m->meta.key_length = 128;
    m->meta.value_length = 128;
    m->meta.vocab_size = 32000;
    m->meta.head_count = 32;
    m->meta.head_count_kv = 32;
    m->meta.bos_token_id = 1;
    m->meta.eos_token_id = 2;
    m->meta.padding_token_id = 0;
    m->meta.add_bos_token = true;
    m->meta.add_eos_token = true;
}

// src/models/vkllm_models_llama2.c:78-183: each key is taken only with the value type the reference accepts
static void parse_meta(const gguf::File &f, vkllm_models_llama2 *m)
{
    struct U32Key
    {
        const char *key;
        uint32_t *dst;
    } u32keys[] = {{"llama.block_count", &m->meta.block_count},
                   {"llama.context_length", &m->meta.context_length},
                   {"llama.embedding_length", &m->meta.embedding_length},
                   {"llama.attention.key_length", &m->meta.key_length},
                   {"llama.attention.value_length", &m->meta.value_length},
                   {"llama.vocab_size", &m->meta.vocab_size},
                   {"llama.attention.head_count", &m->meta.head_count},
                   {"llama.attention.head_count_kv", &m->meta.head_count_kv},
                   {"tokenizer.ggml.bos_token_id", &m->meta.bos_token_id},
                   {"tokenizer.ggml.eos_token_id", &m->meta.eos_token_id},
                   {"tokenizer.ggml.padding_token_id", &m->meta.padding_token_id}};
    for (const gguf::KV &kv : f.kvs)
    {
        for (auto &k : u32keys)
            if (kv.key == k.key && kv.type == gguf::T_UINT32)
                *k.dst = (uint32_t)kv.u64;
        if (kv.key == "llama.rope.freq_base" && kv.type == gguf::T_FLOAT32)
            m->meta.rope_freq_base = (float)kv.f64;
        else if (kv.key == "llama.attention.layer_norm_rms_epsilon" && kv.type == gguf::T_FLOAT32)
            m->meta.layer_norm_rms_epsilon = (float)kv.f64;
        else if (kv.key == "tokenizer.ggml.add_bos_token" && kv.type == gguf::T_BOOL)
            m->meta.add_bos_token = kv.u64 != 0;
        else if (kv.key == "tokenizer.ggml.add_eos_token" && kv.type == gguf::T_BOOL)
            m->meta.add_eos_token = kv.u64 != 0;
    }
    const gguf::KV *toks = f.find("tokenizer.ggml.tokens");
    if (toks && toks->type == gguf::T_ARRAY && toks->arr_type == gguf::T_STRING && toks->arr_len > 0)
    {
        std::vector<std::string> texts = gguf::string_array(*toks);
        std::vector<float> scores;
        std::vector<int32_t> types;
        if (const gguf::KV *s = f.find("tokenizer.ggml.scores"))
            scores = gguf::f32_array(*s);
        if (const gguf::KV *t = f.find("tokenizer.ggml.token_type"))
            types = gguf::i32_array(*t);
        vkllm_array_token_new(&m->meta.tokens, texts.size());
        for (size_t i = 0; i < texts.size(); ++i)
        {
            vkllm_token tok;
            tok.text = strdup(texts[i].c_str());
            tok.score = i < scores.size() ? scores[i] : 0.0f;
            tok.type = i < types.size() ? types[i] : 0;
            vkllm_array_token_append(m->meta.tokens, tok);
        }
    }
}

// a weight tensor whose memory lives in a slab
static vkllm_err_t slab_tensor(vkllm_context *ctx, const char *name, uint32_t rows, uint32_t cols, vkllm_dtype_t dt,
                               void *dev, vkllm_tensor **out)
{
    uint32_t shapes[4] = {1, 1, rows, cols};
    // op REF keeps tensor_new from allocating; the tensor then becomes an ordinary NONE tensor over `dev`
    _CHECK(vkllm_tensor_new(ctx, name, shapes, dt, VKLLM_OP_REF, nullptr, 0, nullptr, 0, false, out));
    (*out)->op = VKLLM_OP_NONE;
    (*out)->data.dev = dev;
    (*out)->data.borrowed = true;
    (*out)->data.valid = true;
    return VKLLM_ERR_OK;
}

static size_t align256(size_t b)
{
    return (b + 255) / 256 * 256;
}

// Lays out the slabs for dims (L, D, F, V) and creates every weight tensor over them.
static vkllm_err_t build_slabs(vkllm_context *ctx, vkllm_models_llama2 *m, ModelPriv *mp)
{
    const size_t D = mp->D, F = mp->F, V = mp->V, L = mp->L;
    size_t per_layer = align256(3 * D * D * 2) + align256(D * D * 2) + align256(2 * F * D * 2) + align256(D * F * 2);
    size_t total = per_layer * L + 2 * align256(V * D * 2);
    HIP_TRY(hipMalloc(&mp->slab, total));
    mp->slab_bytes = total;
    size_t norms = align256(D * 4) * (2 * L + 1);
    HIP_TRY(hipMalloc(&mp->norm_slab, norms));
    char *s = (char *)mp->slab;
    char *n = (char *)mp->norm_slab;
    _CHECK(vkllm_array_block_weights_new(&m->weights.blocks, L));
    mp->layers.resize(L);
    char name[128];
    for (size_t l = 0; l < L; ++l)
    {
        auto *bw = (block_weights *)calloc(1, sizeof(block_weights));
        if (!bw)
            return VKLLM_ERR_ALLOC;
        vkllm_array_block_weights_append(m->weights.blocks, bw);
        ModelPriv::Layer &ly = mp->layers[l];
        ly.wqkv = (uint16_t *)s;
        s += align256(3 * D * D * 2);
        ly.wo = (uint16_t *)s;
        s += align256(D * D * 2);
        ly.wug = (uint16_t *)s;
        s += align256(2 * F * D * 2);
        ly.wd = (uint16_t *)s;
        s += align256(D * F * 2);
        ly.attn_norm = (float *)n;
        n += align256(D * 4);
        ly.ffn_norm = (float *)n;
        n += align256(D * 4);
        ly.kc = ly.vc = nullptr;
#define MK(_field, _suffix, _rows, _cols, _dt, _ptr)                                                                \
    snprintf(name, sizeof(name), "blk.%zu." _suffix, l);                                                            \
    _CHECK(slab_tensor(ctx, name, (uint32_t)(_rows), (uint32_t)(_cols), _dt, (void *)(_ptr), &bw->_field))
        MK(attn_norm_weight, "attn_norm.weight", 1, D, vkllm_dtype_float32, ly.attn_norm);
        MK(WQ, "attn_q.weight", D, D, vkllm_dtype_float16, ly.wqkv);
        MK(WK, "attn_k.weight", D, D, vkllm_dtype_float16, ly.wqkv + D * D);
        MK(WV, "attn_v.weight", D, D, vkllm_dtype_float16, ly.wqkv + 2 * D * D);
        MK(WO, "attn_output.weight", D, D, vkllm_dtype_float16, ly.wo);
        MK(ffn_norm_weight, "ffn_norm.weight", 1, D, vkllm_dtype_float32, ly.ffn_norm);
        MK(WU, "ffn_up.weight", F, D, vkllm_dtype_float16, ly.wug);
        MK(WG, "ffn_gate.weight", F, D, vkllm_dtype_float16, ly.wug + F * D);
        MK(WD, "ffn_down.weight", D, F, vkllm_dtype_float16, ly.wd);
#undef MK
    }
    mp->embd = (uint16_t *)s;
    s += align256(V * D * 2);
    mp->out_w = (uint16_t *)s;
    mp->out_norm = (float *)n;
    _CHECK(slab_tensor(ctx, "token_embd.weight", (uint32_t)V, (uint32_t)D, vkllm_dtype_float16, mp->embd,
                       &m->weights.tok_embed_weights));
    _CHECK(slab_tensor(ctx, "output.weight", (uint32_t)V, (uint32_t)D, vkllm_dtype_float16, mp->out_w,
                       &m->weights.output_weight));
    _CHECK(slab_tensor(ctx, "output_norm.weight", 1, (uint32_t)D, vkllm_dtype_float32, mp->out_norm,
                       &m->weights.output_norm_weight));
    return VKLLM_ERR_OK;
}

void model_bind_kv(vkllm_context *ctx, vkllm_models_llama2 *model)
{
    ModelPriv *mp = model_priv(model);
    vkllm_kvcache *kv = model->weights.kvcache;
    for (size_t l = 0; l < mp->layers.size() && kv && l < kv->kcaches->used_n; ++l)
    {
        mp->layers[l].kc = (uint16_t *)tensor_dev(ctx, kv->kcaches->data[l]);
        mp->layers[l].vc = (uint16_t *)tensor_dev(ctx, kv->vcaches->data[l]);
    }
}

// src/models/vkllm_models_llama2.c:243-253
static vkllm_err_t create_kvcache(vkllm_context *ctx, vkllm_models_llama2 *m)
{
    _CHECK_ARGS(m->weights.blocks && m->weights.blocks->used_n > 0 && m->weights.blocks->data[0]->WK);
    uint32_t khd = m->weights.blocks->data[0]->WK->shapes[3] / m->meta.head_count;
    uint32_t vhd = m->weights.blocks->data[0]->WV->shapes[3] / m->meta.head_count;
    uint32_t ks[4] = {1, m->meta.head_count, m->meta.context_length, khd};
    uint32_t vs[4] = {1, m->meta.head_count, m->meta.context_length, vhd};
    return vkllm_kvcache_new(ctx, ks, vs, m->meta.block_count, &m->weights.kvcache);
}

static void finish_priv(vkllm_models_llama2 *m, ModelPriv *mp)
{
    mp->H = m->meta.head_count;
    mp->hd = mp->H ? mp->D / mp->H : 0;
    mp->ctx = m->meta.context_length;
    mp->eps = m->meta.layer_norm_rms_epsilon;
    mp->theta = m->meta.rope_freq_base;
    mp->pad_id = m->meta.padding_token_id;
    mp->rope_freqs.resize(mp->hd / 2);
    for (uint32_t w = 0; w < mp->hd / 2; ++w)
        mp->rope_freqs[w] = powf(mp->theta, (float)(2 * w) / (float)mp->hd);
    // the fused kernels move 16-byte vectors along rows and give each head its own wave group
    mp->fused_ok = mp->slab && mp->H > 0 && mp->D == mp->H * mp->hd && mp->hd % 8 == 0 && mp->hd <= 256 &&
                   mp->D % 8 == 0 && mp->F % 8 == 0 && mp->V == m->meta.vocab_size &&
                   mp->L == m->meta.block_count && m->weights.kvcache &&
                   m->weights.kvcache->kcaches->used_n == mp->L;
}

// copies host bytes into device memory through a pinned bounce buffer
static vkllm_err_t upload_bytes(vkllm_context *ctx, void *dst, const void *src, size_t bytes, void *pinned,
                                size_t pinned_bytes)
{
    hipStream_t st = ctx->device->stream;
    for (size_t off = 0; off < bytes; off += pinned_bytes)
    {
        size_t n = bytes - off < pinned_bytes ? bytes - off : pinned_bytes;
        memcpy(pinned, (const char *)src + off, n);
        HIP_TRY(hipMemcpyAsync((char *)dst + off, pinned, n, hipMemcpyHostToDevice, st));
        HIP_TRY(hipStreamSynchronize(st));
    }
    return VKLLM_ERR_OK;
}

// tensors in the file that go into the slab, by name
static void *slab_dst(ModelPriv *mp, vkllm_models_llama2 *m, const gguf::TensorInfo &t, uint64_t rows, uint64_t cols,
                      bool is_norm)
{
    (void)m;
    const uint64_t D = mp->D, F = mp->F, V = mp->V;
    if (t.name == "token_embd.weight")
        return rows == V && cols == D && t.type == gguf::GGML_F16 ? mp->embd : nullptr;
    if (t.name == "output.weight")
        return rows == V && cols == D && t.type == gguf::GGML_F16 ? mp->out_w : nullptr;
    if (t.name == "output_norm.weight")
        return rows == 1 && cols == D && t.type == gguf::GGML_F32 ? mp->out_norm : nullptr;
    unsigned l = 0;
    char rest[96];
    if (sscanf(t.name.c_str(), "blk.%u.%95s", &l, rest) != 2 || l >= mp->L)
        return nullptr;
    const ModelPriv::Layer &ly = mp->layers[l];
    std::string r(rest);
    (void)is_norm;
    if (r == "attn_norm.weight")
        return rows == 1 && cols == D && t.type == gguf::GGML_F32 ? ly.attn_norm : nullptr;
    if (r == "ffn_norm.weight")
        return rows == 1 && cols == D && t.type == gguf::GGML_F32 ? ly.ffn_norm : nullptr;
    if (t.type != gguf::GGML_F16)
        return nullptr;
    if (r == "attn_q.weight" && rows == D && cols == D)
        return ly.wqkv;
    if (r == "attn_k.weight" && rows == D && cols == D)
        return ly.wqkv + D * D;
    if (r == "attn_v.weight" && rows == D && cols == D)
        return ly.wqkv + 2 * D * D;
    if (r == "attn_output.weight" && rows == D && cols == D)
        return ly.wo;
    if (r == "ffn_up.weight" && rows == F && cols == D)
        return ly.wug;
    if (r == "ffn_gate.weight" && rows == F && cols == D)
        return ly.wug + F * D;
    if (r == "ffn_down.weight" && rows == D && cols == F)
        return ly.wd;
    return nullptr;
}

// standalone tensor (the reference's create_tensor_from_gguf, src/models/vkllm_models_llama2.c:189-222):
// F32 -> float32, F16 -> float16, any other encoding is read as float16 bytes
static vkllm_err_t standalone_tensor(vkllm_context *ctx, vkllm_commands *cmds, const gguf::TensorInfo &t,
                                     vkllm_tensor **out)
{
    vkllm_dtype_t dt = t.type == gguf::GGML_F32 ? vkllm_dtype_float32 : vkllm_dtype_float16;
    if (t.type != gguf::GGML_F32 && t.type != gguf::GGML_F16)
        log_error("tensor %s has GGML type %u; reading its bytes as float16 like the reference", t.name.c_str(),
                  t.type);
    uint32_t shapes[4] = {1, 1, 1, 1};
    for (uint32_t i = 0; i < t.n_dims && i < 4; ++i)
        shapes[3 - i] = (uint32_t)t.ne[i];
    _CHECK(vkllm_tensor_new(ctx, t.name.c_str(), shapes, dt, VKLLM_OP_NONE, nullptr, 0, nullptr, 0, false, out));
    size_t n = t.bytes < (*out)->bytes ? t.bytes : (*out)->bytes;
    return vkllm_commands_upload(ctx, cmds, *out, t.data, n);
}

static vkllm_err_t load_standalone(vkllm_context *ctx, vkllm_models_llama2 *m, const gguf::File &f)
{
    vkllm_commands *cmds = nullptr;
    _CHECK(vkllm_commands_new(ctx, &cmds));
    vkllm_err_t rc = vkllm_array_block_weights_new(&m->weights.blocks, m->meta.block_count);
    for (const gguf::TensorInfo &t : f.tensors)
    {
        if (rc != VKLLM_ERR_OK)
            break;
        vkllm_tensor **slot = nullptr;
        unsigned l = 0;
        char rest[96];
        if (t.name == "token_embd.weight")
            slot = &m->weights.tok_embed_weights;
        else if (t.name == "output_norm.weight")
            slot = &m->weights.output_norm_weight;
        else if (t.name == "output.weight")
            slot = &m->weights.output_weight;
        else if (sscanf(t.name.c_str(), "blk.%u.%95s", &l, rest) == 2 && l < m->meta.block_count)
        {
            while (m->weights.blocks->used_n <= l)
                vkllm_array_block_weights_append(m->weights.blocks,
                                                 (block_weights *)calloc(1, sizeof(block_weights)));
            block_weights *bw = m->weights.blocks->data[l];
            std::string r(rest);
            if (r == "attn_norm.weight")
                slot = &bw->attn_norm_weight;
            else if (r == "ffn_norm.weight")
                slot = &bw->ffn_norm_weight;
            else if (r == "attn_q.weight")
                slot = &bw->WQ;
            else if (r == "attn_k.weight")
                slot = &bw->WK;
            else if (r == "attn_v.weight")
                slot = &bw->WV;
            else if (r == "attn_output.weight")
                slot = &bw->WO;
            else if (r == "ffn_gate.weight")
                slot = &bw->WG;
            else if (r == "ffn_up.weight")
                slot = &bw->WU;
            else if (r == "ffn_down.weight")
                slot = &bw->WD;
        }
        if (slot && !*slot)
            rc = standalone_tensor(ctx, cmds, t, slot);
    }
    vkllm_commands_free(ctx, cmds);
    return rc;
}

extern "C" vkllm_err_t vkllm_models_llama2_free(struct vkllm_context *context, struct vkllm_models_llama2 *model);

// Every weight the graph reads was found in the file. The reference leaves a missing one NULL and the graph build
// then dereferences it; here the load fails instead and names the first missing tensor.
static bool all_weights_present(const vkllm_models_llama2 *m, const char *file)
{
    const char *missing = nullptr;
    unsigned layer = 0;
    if (!m->weights.tok_embed_weights)
        missing = "token_embd.weight";
    else if (!m->weights.output_norm_weight)
        missing = "output_norm.weight";
    else if (!m->weights.output_weight)
        missing = "output.weight";
    for (uint32_t l = 0; !missing && m->weights.blocks && l < m->weights.blocks->used_n; ++l)
    {
        const block_weights *b = m->weights.blocks->data[l];
        layer = l;
        if (!b->attn_norm_weight)
            missing = "attn_norm.weight";
        else if (!b->ffn_norm_weight)
            missing = "ffn_norm.weight";
        else if (!b->WQ || !b->WK || !b->WV || !b->WO)
            missing = "an attention weight";
        else if (!b->WU || !b->WG || !b->WD)
            missing = "an ffn weight";
    }
    if (!missing && (!m->weights.blocks || m->weights.blocks->used_n != m->meta.block_count))
        missing = "a block";
    if (missing)
    {
        log_error("gguf %s lacks %s (block %u)", file, missing, layer);
        return false;
    }
    return true;
}

extern "C" vkllm_err_t vkllm_models_llama2_load(struct vkllm_context *context, struct vkllm_models_llama2 *model,
                                                const char *file)
{
    DeviceScope device_scope(context);
    _CHECK_ARGS(context && model && file);
    memset(model, 0, sizeof(*model));
    gguf::File f;
    std::string err;
    if (!f.open(file, &err))
    {
        log_error("failed to open gguf file: %s (%s)", file, err.c_str());
        return VKLLM_ERR_ARGS;
    }
    set_defaults(model);
    parse_meta(f, model);
    auto *mp = new ModelPriv();
    model->priv = mp;

    // dims from the tensors themselves; the slab layout needs all of them consistent
    const gguf::TensorInfo *embd = nullptr, *up0 = nullptr;
    for (const gguf::TensorInfo &t : f.tensors)
    {
        if (t.name == "token_embd.weight")
            embd = &t;
        else if (t.name == "blk.0.ffn_up.weight")
            up0 = &t;
    }
    bool slabbed = embd && up0 && embd->n_dims == 2 && up0->n_dims == 2;
    if (slabbed)
    {
        mp->D = (uint32_t)embd->ne[0];
        mp->V = (uint32_t)embd->ne[1];
        mp->F = (uint32_t)up0->ne[1];
        mp->L = model->meta.block_count;
        // every expected tensor must be present with its slab shape and type
        size_t expected = 9 * (size_t)mp->L + 3, matched = 0;
        // slab regions already claimed: a name repeated in the file must not count twice (its region would be
        // written twice while another one stayed uninitialised)
        std::unordered_set<const void *> claimed;
        vkllm_err_t rc = build_slabs(context, model, mp);
        if (rc != VKLLM_ERR_OK)
        {
            vkllm_models_llama2_free(context, model);
            return rc;
        }
        std::vector<const gguf::TensorInfo *> plan(f.tensors.size(), nullptr);
        std::vector<void *> dst(f.tensors.size(), nullptr);
        for (size_t i = 0; i < f.tensors.size(); ++i)
        {
            const gguf::TensorInfo &t = f.tensors[i];
            uint64_t cols = t.ne[0], rows = t.n_dims >= 2 ? t.ne[1] : 1;
            if (t.n_dims > 2)
                continue;
            void *d = slab_dst(mp, model, t, rows, cols, false);
            if (d && claimed.insert(d).second)
            {
                dst[i] = d;
                matched++;
            }
        }
        if (matched == expected)
        {
            void *pinned = nullptr;
            const size_t pinned_bytes = 64u << 20;
            if (hipHostMalloc(&pinned, pinned_bytes, hipHostMallocDefault) != hipSuccess)
            {
                (void)hipGetLastError();
                vkllm_models_llama2_free(context, model);
                return VKLLM_ERR_ALLOC;
            }
            vkllm_err_t urc = VKLLM_ERR_OK;
            for (size_t i = 0; i < f.tensors.size() && urc == VKLLM_ERR_OK; ++i)
                if (dst[i])
                    urc = upload_bytes(context, dst[i], f.tensors[i].data, f.tensors[i].bytes, pinned, pinned_bytes);
            (void)hipHostFree(pinned);
            if (urc != VKLLM_ERR_OK)
            {
                vkllm_models_llama2_free(context, model);
                return urc;
            }
        }
        else
        {
            log_info("gguf %s does not match the fp16 slab layout (%zu of %zu tensors); loading tensor by tensor",
                     file, matched, expected);
            // discard the slab plan
            ModelPriv *keep = mp;
            model->priv = nullptr;
            vkllm_models_llama2_free(context, model);
            memset(model, 0, sizeof(*model));
            set_defaults(model);
            parse_meta(f, model);
            (void)keep;
            mp = new ModelPriv();
            model->priv = mp;
            if (keep->slab)
                (void)hipFree(keep->slab);
            if (keep->norm_slab)
                (void)hipFree(keep->norm_slab);
            delete keep;
            slabbed = false;
        }
    }
    if (!slabbed)
    {
        vkllm_err_t rc = load_standalone(context, model, f);
        if (rc == VKLLM_ERR_OK && !all_weights_present(model, file))
            rc = VKLLM_ERR_ARGS;
        if (rc != VKLLM_ERR_OK)
        {
            vkllm_models_llama2_free(context, model);
            return rc;
        }
    }
    vkllm_err_t rc = create_kvcache(context, model);
    if (rc != VKLLM_ERR_OK)
    {
        vkllm_models_llama2_free(context, model);
        return rc;
    }
    finish_priv(model, mp);
    model_bind_kv(context, model);
    HIP_TRY(hipStreamSynchronize(context->device->stream));
    return VKLLM_ERR_OK;
}

extern "C" vkllm_err_t vkllm_models_llama2_init_random(struct vkllm_context *context,
                                                       struct vkllm_models_llama2 *model,
                                                       const struct vkllm_llama2_config *cfg, uint64_t seed)
{
    DeviceScope device_scope(context);
    _CHECK_ARGS(context && model && cfg);
    _CHECK_ARGS(cfg->block_count > 0 && cfg->embedding_length > 0 && cfg->head_count > 0 &&
                cfg->feed_forward_length > 0 && cfg->vocab_size > 0 && cfg->context_length > 0);
    memset(model, 0, sizeof(*model));
    set_defaults(model);
    model->meta.block_count = cfg->block_count;
    model->meta.context_length = cfg->context_length;
    model->meta.embedding_length = cfg->embedding_length;
    model->meta.head_count = model->meta.head_count_kv = cfg->head_count;
    model->meta.key_length = model->meta.value_length = cfg->embedding_length / cfg->head_count;
    model->meta.vocab_size = cfg->vocab_size;
    model->meta.rope_freq_base = cfg->rope_freq_base;
    model->meta.layer_norm_rms_epsilon = cfg->layer_norm_rms_epsilon;
    model->meta.add_eos_token = false;
    auto *mp = new ModelPriv();
    model->priv = mp;
    mp->L = cfg->block_count;
    mp->D = cfg->embedding_length;
    mp->F = cfg->feed_forward_length;
    mp->V = cfg->vocab_size;
    vkllm_err_t rc = build_slabs(context, model, mp);
    if (rc != VKLLM_ERR_OK)
    {
        vkllm_models_llama2_free(context, model);
        return rc;
    }
    // tensor ids of the random-init GGUF definition: token_embd 0; block l: attn_norm, attn_q, attn_k, attn_v,
    // attn_output, ffn_norm, ffn_gate, ffn_up, ffn_down = 1+9l..9+9l; output_norm 1+9L; output 2+9L
    auto key = [seed](uint64_t id) {
        uint64_t z = seed + (id + 1) * 0x9E3779B97F4A7C15ull;
        z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
        z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
        return z ^ (z >> 31);
    };
    hipStream_t st = context->device->stream;
    const uint64_t D = mp->D, F = mp->F, V = mp->V, L = mp->L;
    const float sd = cfg->weight_std;
#define RND(_ptr, _count, _id) HIP_TRY(vk::launch_random_f16(st, (uint16_t *)(_ptr), (_count), key(_id), sd))
#define ONES(_ptr, _count) HIP_TRY(vk::launch_fill_f32(st, (float *)(_ptr), (_count), 1.0f))
    RND(mp->embd, V * D, 0);
    for (uint64_t l = 0; l < L; ++l)
    {
        const ModelPriv::Layer &ly = mp->layers[l];
        const uint64_t b = 1 + 9 * l;
        ONES(ly.attn_norm, D);
        RND(ly.wqkv, D * D, b + 1);
        RND(ly.wqkv + D * D, D * D, b + 2);
        RND(ly.wqkv + 2 * D * D, D * D, b + 3);
        RND(ly.wo, D * D, b + 4);
        ONES(ly.ffn_norm, D);
        RND(ly.wug + F * D, F * D, b + 6); // gate
        RND(ly.wug, F * D, b + 7);         // up
        RND(ly.wd, D * F, b + 8);
    }
    ONES(mp->out_norm, D);
    RND(mp->out_w, V * D, 2 + 9 * L);
#undef RND
#undef ONES
    rc = create_kvcache(context, model);
    if (rc != VKLLM_ERR_OK)
    {
        vkllm_models_llama2_free(context, model);
        return rc;
    }
    finish_priv(model, mp);
    model_bind_kv(context, model);
    HIP_TRY(hipStreamSynchronize(st));
    return VKLLM_ERR_OK;
}

extern "C" vkllm_err_t vkllm_models_llama2_free(struct vkllm_context *context, struct vkllm_models_llama2 *model)
{
    DeviceScope device_scope(context);
    _CHECK_ARGS(context && model);
    (void)hipStreamSynchronize(context->device->stream);
    if (model->meta.tokens)
    {
        for (size_t i = 0; i < model->meta.tokens->used_n; ++i)
            free(model->meta.tokens->data[i].text);
        vkllm_array_token_free(model->meta.tokens);
        model->meta.tokens = nullptr;
    }
    vkllm_tensor *singles[3] = {model->weights.tok_embed_weights, model->weights.output_norm_weight,
                                model->weights.output_weight};
    for (vkllm_tensor *t : singles)
        if (t)
            vkllm_tensor_free(context, t);
    model->weights.tok_embed_weights = model->weights.output_norm_weight = model->weights.output_weight = nullptr;
    if (model->weights.blocks)
    {
        for (size_t i = 0; i < model->weights.blocks->used_n; ++i)
        {
            block_weights *bw = model->weights.blocks->data[i];
            if (!bw)
                continue;
            vkllm_tensor *ts[9] = {bw->attn_norm_weight, bw->ffn_norm_weight, bw->WQ, bw->WK, bw->WV,
                                   bw->WO,               bw->WU,              bw->WG, bw->WD};
            for (vkllm_tensor *t : ts)
                if (t)
                    vkllm_tensor_free(context, t);
            free(bw);
        }
        vkllm_array_block_weights_free(model->weights.blocks);
        model->weights.blocks = nullptr;
    }
    if (model->weights.kvcache)
    {
        vkllm_kvcache_free(context, model->weights.kvcache);
        model->weights.kvcache = nullptr;
    }
    ModelPriv *mp = model_priv(model);
    if (mp)
    {
        fused_model_release(context, model);
        if (mp->slab)
            (void)hipFree(mp->slab);
        if (mp->norm_slab)
            (void)hipFree(mp->norm_slab);
        delete mp;
        model->priv = nullptr;
    }
    return VKLLM_ERR_OK;
}

// =============================================================================================================
// graph construction: src/models/vkllm_llama2_layers.c:13-354, src/models/vkllm_models_llama2.c:488-602

// dst = a + "." + b (truncated to n - 1 bytes): node names are built for every node of every step, and a formatted
// print per name costs more than the rest of building the node
static void scope_name(char *dst, size_t n, const char *a, const char *b)
{
    const size_t la = strnlen(a, n - 1);
    memcpy(dst, a, la);
    size_t at = la;
    if (at < n - 1)
        dst[at++] = '.';
    const size_t lb = strnlen(b, n - 1 - at);
    memcpy(dst + at, b, lb);
    dst[at + lb] = '\0';
}

extern "C" vkllm_err_t vkllm_llama2_build_ffn_layer(struct vkllm_context *context, struct vkllm_graph *graph,
                                                    struct vkllm_tensor *input,
                                                    struct vkllm_llama2_ffn_layer_params params, uint32_t block_idx)
{
    DeviceScope device_scope(context);
    _CHECK_ARGS(context && graph && input && params.WD && params.WG && params.WU);
    const uint32_t batch = input->shapes[0], channel = input->shapes[1], seq = input->shapes[2];
    const uint32_t up_dim = params.WU->shapes[2];
    char name[64], scope[128];
    snprintf(name, sizeof(name), "block.%u.ffn", block_idx);
    vkllm_tensor *t = nullptr;

    vkllm_tensor *norm_srcs[] = {input, params.norm_weight};
    vkllm_op_rmsnorm_params np = {params.norm_power, params.norm_eps};
    scope_name(scope, sizeof(scope), name, "norm");
    _CHECK(vkllm_tensor_new(context, scope, input->shapes, input->dtype, VKLLM_OP_RMSNORM, norm_srcs, 2, &np,
                            sizeof(np), false, &t));
    vkllm_tensor *norm = t;
    if (vkllm_graph_add_node(context, graph, norm) != VKLLM_ERR_OK)
        return vkllm_tensor_free(context, norm), VKLLM_ERR_ALLOC;

    uint32_t up_shapes[4] = {batch, channel, seq, up_dim};
    vkllm_op_matmul_params mp0 = {1.0f, 0}, mp1 = {1.0f, 1};
    vkllm_tensor *up_srcs[] = {norm, params.WU};
    scope_name(scope, sizeof(scope), name, "up");
    _CHECK(vkllm_tensor_new(context, scope, up_shapes, norm->dtype, VKLLM_OP_MATMUL, up_srcs, 2, &mp0, sizeof(mp0),
                            false, &t));
    vkllm_tensor *up = t;
    if (vkllm_graph_add_node(context, graph, up) != VKLLM_ERR_OK)
        return vkllm_tensor_free(context, up), VKLLM_ERR_ALLOC;

    vkllm_tensor *gate_srcs[] = {norm, params.WG};
    scope_name(scope, sizeof(scope), name, "gate");
    _CHECK(vkllm_tensor_new(context, scope, up_shapes, norm->dtype, VKLLM_OP_MATMUL, gate_srcs, 2, &mp1, sizeof(mp1),
                            false, &t));
    vkllm_tensor *gate = t;
    if (vkllm_graph_add_node(context, graph, gate) != VKLLM_ERR_OK)
        return vkllm_tensor_free(context, gate), VKLLM_ERR_ALLOC;

    int32_t mul_op = 2;
    vkllm_tensor *mul_srcs[] = {up, gate};
    scope_name(scope, sizeof(scope), name, "mul");
    _CHECK(vkllm_tensor_new(context, scope, up_shapes, gate->dtype, VKLLM_OP_BIN, mul_srcs, 2, &mul_op,
                            sizeof(mul_op), false, &t));
    vkllm_tensor *gate_mul = t;
    if (vkllm_graph_add_node(context, graph, gate_mul) != VKLLM_ERR_OK)
        return vkllm_tensor_free(context, gate_mul), VKLLM_ERR_ALLOC;

    uint32_t down_shapes[4] = {batch, channel, seq, params.WD->shapes[2]};
    vkllm_tensor *down_srcs[] = {gate_mul, params.WD};
    scope_name(scope, sizeof(scope), name, "down");
    _CHECK(vkllm_tensor_new(context, scope, down_shapes, gate_mul->dtype, VKLLM_OP_MATMUL, down_srcs, 2, &mp0,
                            sizeof(mp0), false, &t));
    vkllm_tensor *down = t;
    if (vkllm_graph_add_node(context, graph, down) != VKLLM_ERR_OK)
        return vkllm_tensor_free(context, down), VKLLM_ERR_ALLOC;

    int32_t add_op = 0;
    vkllm_tensor *add_srcs[] = {input, down};
    scope_name(scope, sizeof(scope), name, "add");
    _CHECK(vkllm_tensor_new(context, scope, input->shapes, input->dtype, VKLLM_OP_BIN, add_srcs, 2, &add_op,
                            sizeof(add_op), false, &t));
    if (vkllm_graph_add_node(context, graph, t) != VKLLM_ERR_OK)
        return vkllm_tensor_free(context, t), VKLLM_ERR_ALLOC;
    return VKLLM_ERR_OK;
}

// adds `t` to the graph or frees it
#define ADD_OR_FREE(_t)                                                                                             \
    do                                                                                                              \
    {                                                                                                               \
        if (vkllm_graph_add_node(context, graph, (_t)) != VKLLM_ERR_OK)                                             \
        {                                                                                                           \
            vkllm_tensor_free(context, (_t));                                                                       \
            return VKLLM_ERR_ALLOC;                                                                                 \
        }                                                                                                           \
    } while (0)

extern "C" vkllm_err_t vkllm_llama2_build_self_attn_layer(struct vkllm_context *context, struct vkllm_graph *graph,
                                                          struct vkllm_kvcache *kvcache, struct vkllm_tensor *input,
                                                          struct vkllm_llama2_self_attn_layer_params params,
                                                          uint32_t block_idx)
{
    DeviceScope device_scope(context);
    _CHECK_ARGS(context && graph && input && params.WQ && params.WK && params.WV);
    vkllm_op_rope_params rope = {params.offsets, params.freq_base, false};
    const uint32_t hidden = params.WQ->shapes[3], nhd = params.WQ->shapes[2];
    _CHECK_ARGS(params.num_head > 0 && nhd % params.num_head == 0);
    const uint32_t hd = nhd / params.num_head;
    _CHECK_ARGS(params.WK->shapes[0] == 1 && params.WK->shapes[1] == 1);
    _CHECK_ARGS(params.WV->shapes[0] == 1 && params.WV->shapes[1] == 1);
    _CHECK_ARGS(params.WK->shapes[2] == nhd && params.WK->shapes[3] == hidden);
    _CHECK_ARGS(params.WV->shapes[2] == nhd && params.WV->shapes[3] == hidden);
    const uint32_t batch = input->shapes[0], seq = input->shapes[2];
    _CHECK_ARGS(input->shapes[3] == hidden);
    char name[64], scope[128];
    snprintf(name, sizeof(name), "block.%u.attn", block_idx);
    vkllm_tensor *t = nullptr;

    vkllm_tensor *norm_srcs[] = {input, params.norm_weight};
    vkllm_op_rmsnorm_params np = {params.norm_power, params.norm_eps};
    scope_name(scope, sizeof(scope), name, "norm");
    _CHECK(vkllm_tensor_new(context, scope, input->shapes, input->dtype, VKLLM_OP_RMSNORM, norm_srcs, 2, &np,
                            sizeof(np), false, &t));
    vkllm_tensor *norm = t;
    ADD_OR_FREE(norm);

    vkllm_op_matmul_params mm = {1.0f, 0};
    uint32_t qkv_shapes[4] = {batch, 1, seq, nhd};
    vkllm_tensor *proj[3];
    vkllm_tensor *W[3] = {params.WQ, params.WK, params.WV};
    const char *pn[3] = {"Q", "K", "V"};
    for (int i = 0; i < 3; ++i)
    {
        vkllm_tensor *srcs[] = {norm, W[i]};
        scope_name(scope, sizeof(scope), name, pn[i]);
        _CHECK(vkllm_tensor_new(context, scope, qkv_shapes, norm->dtype, VKLLM_OP_MATMUL, srcs, 2, &mm, sizeof(mm),
                                false, &t));
        proj[i] = t;
        ADD_OR_FREE(t);
    }

    // [batch, 1, seq, H*hd] -> [batch, seq, H, hd] -> [batch, H, seq, hd] views
    uint32_t split[4] = {batch, seq, params.num_head, hd};
    uint32_t axis[4] = {0, 2, 1, 3};
    vkllm_tensor *refs[3];
    for (int i = 0; i < 3; ++i)
    {
        _CHECK(vkllm_tensor_copy_ref(context, proj[i], &refs[i]));
        vkllm_err_t rc = vkllm_tensor_reshape(context, refs[i], split);
        if (rc != VKLLM_ERR_OK)
        {
            vkllm_tensor_free(context, refs[i]);
            return rc;
        }
        ADD_OR_FREE(refs[i]);
        _CHECK(vkllm_tensor_permute(context, refs[i], axis));
    }
    vkllm_tensor *Q_ref = refs[0], *K_ref = refs[1], *V_ref = refs[2];

    scope_name(scope, sizeof(scope), name, "RQ");
    _CHECK(vkllm_tensor_new(context, scope, Q_ref->shapes, Q_ref->dtype, VKLLM_OP_ROPE, &Q_ref, 1, &rope,
                            sizeof(rope), false, &t));
    vkllm_tensor *RQ = t;
    ADD_OR_FREE(RQ);
    scope_name(scope, sizeof(scope), name, "RK");
    _CHECK(vkllm_tensor_new(context, scope, K_ref->shapes, K_ref->dtype, VKLLM_OP_ROPE, &K_ref, 1, &rope,
                            sizeof(rope), false, &t));
    vkllm_tensor *RK = t;
    ADD_OR_FREE(RK);

    // RK and V_ref become views [batch, H, offset + seq, hd] of this layer's caches
    _CHECK(vkllm_kvcache_update(context, kvcache, &RK, &V_ref, block_idx, params.offsets));

    const uint32_t key_num = RK->shapes[2];
    uint32_t scores_shapes[4] = {batch, params.num_head, seq, key_num};
    vkllm_op_matmul_params smm = {1.0f / sqrtf((float)hd), 0};
    vkllm_tensor *scores_srcs[] = {RQ, RK};
    scope_name(scope, sizeof(scope), name, "scores");
    _CHECK(vkllm_tensor_new(context, scope, scores_shapes, input->dtype, VKLLM_OP_MATMUL, scores_srcs, 2, &smm,
                            sizeof(smm), false, &t));
    vkllm_tensor *scores = t;
    ADD_OR_FREE(scores);

    vkllm_op_softmax_params sp = {1, rope.offset};
    scope_name(scope, sizeof(scope), name, "attn_weights");
    _CHECK(vkllm_tensor_new(context, scope, scores_shapes, input->dtype, VKLLM_OP_SOFTMAX, &scores, 1, &sp,
                            sizeof(sp), false, &t));
    vkllm_tensor *attn_w = t;
    ADD_OR_FREE(attn_w);

    uint32_t out_shapes[4] = {batch, params.num_head, seq, hd};
    vkllm_tensor *out_srcs[] = {attn_w, V_ref};
    _CHECK(vkllm_tensor_new(context, name, out_shapes, input->dtype, VKLLM_OP_MATMUL, out_srcs, 2, &mm, sizeof(mm),
                            false, &t));
    vkllm_tensor *output = t;
    ADD_OR_FREE(output);

    vkllm_tensor *output_ref = nullptr;
    _CHECK(vkllm_tensor_copy_ref(context, output, &output_ref));
    if (vkllm_tensor_permute(context, output_ref, axis) != VKLLM_ERR_OK)
    {
        vkllm_tensor_free(context, output_ref);
        return VKLLM_ERR_ARGS;
    }
    ADD_OR_FREE(output_ref);

    scope_name(scope, sizeof(scope), name, "concated_heads");
    _CHECK(vkllm_tensor_new(context, scope, output_ref->shapes, output_ref->dtype, VKLLM_OP_COPY, &output_ref, 1,
                            nullptr, 0, false, &t));
    vkllm_tensor *concat = t;
    ADD_OR_FREE(concat);
    vkllm_tensor *concat_ref = nullptr;
    _CHECK(vkllm_tensor_copy_ref(context, concat, &concat_ref));
    ADD_OR_FREE(concat_ref);
    uint32_t merged[4] = {batch, 1, seq, nhd};
    _CHECK(vkllm_tensor_reshape(context, concat_ref, merged));

    uint32_t fo_shapes[4] = {batch, 1, seq, hidden};
    vkllm_tensor *fo_srcs[] = {concat_ref, params.WO};
    vkllm_op_matmul_params om = {1.0f, 0};
    scope_name(scope, sizeof(scope), name, "final_output");
    _CHECK(vkllm_tensor_new(context, scope, fo_shapes, concat->dtype, VKLLM_OP_MATMUL, fo_srcs, 2, &om, sizeof(om),
                            false, &t));
    vkllm_tensor *fo = t;
    ADD_OR_FREE(fo);

    int32_t add_op = 0;
    vkllm_tensor *add_srcs[] = {input, fo};
    scope_name(scope, sizeof(scope), name, "final_output_add");
    _CHECK(vkllm_tensor_new(context, scope, fo->shapes, fo->dtype, VKLLM_OP_BIN, add_srcs, 2, &add_op, sizeof(add_op),
                            false, &t));
    ADD_OR_FREE(t);
    return VKLLM_ERR_OK;
}

extern "C" vkllm_err_t vkllm_llama2_build_transformer_block(struct vkllm_context *context, struct vkllm_graph *graph,
                                                            struct vkllm_kvcache *kvcache, struct vkllm_tensor *input,
                                                            struct vkllm_llama2_transformer_block_params params,
                                                            uint32_t block_idx)
{
    DeviceScope device_scope(context);
    _CHECK_ARGS(context && graph && input);
    _CHECK(vkllm_llama2_build_self_attn_layer(context, graph, kvcache, input, params.attn, block_idx));
    vkllm_tensor *attn_out = graph->nodes->data[graph->nodes->used_n - 1];
    return vkllm_llama2_build_ffn_layer(context, graph, attn_out, params.ffn, block_idx);
}

static vkllm_err_t build_graph_body(vkllm_context *context, vkllm_models_llama2 *model, vkllm_tensor *input_toks,
                                    vkllm_graph *graph, uint32_t offsets)
{
    const uint32_t batch = input_toks->shapes[0], seq = input_toks->shapes[3];
    const uint32_t hidden_dim = model->meta.embedding_length, vocab = model->meta.vocab_size;
    _CHECK(vkllm_graph_add_input(context, graph, input_toks));
    vkllm_tensor *t = nullptr;
    uint32_t embed_shapes[4] = {batch, 1, seq, hidden_dim};
    vkllm_tensor *embed_srcs[] = {input_toks, model->weights.tok_embed_weights};
    uint32_t unk = model->meta.padding_token_id;
    _CHECK(vkllm_tensor_new(context, "embedded", embed_shapes, vkllm_dtype_float16, VKLLM_OP_EMBEDDING, embed_srcs, 2,
                            &unk, sizeof(unk), false, &t));
    if (vkllm_graph_add_node(context, graph, t) != VKLLM_ERR_OK)
        return vkllm_tensor_free(context, t), VKLLM_ERR_ALLOC;
    vkllm_tensor *hidden = t;
    for (uint32_t i = 0; i < model->meta.block_count && i < model->weights.blocks->used_n; ++i)
    {
        block_weights *bw = model->weights.blocks->data[i];
        if (!bw)
            return VKLLM_ERR_ARGS;
        vkllm_llama2_transformer_block_params bp;
        bp.attn.WK = bw->WK;
        bp.attn.WQ = bw->WQ;
        bp.attn.WV = bw->WV;
        bp.attn.WO = bw->WO;
        bp.attn.norm_weight = bw->attn_norm_weight;
        bp.attn.norm_power = 2.0f;
        bp.attn.norm_eps = model->meta.layer_norm_rms_epsilon;
        bp.attn.freq_base = model->meta.rope_freq_base;
        bp.attn.offsets = offsets;
        bp.attn.num_head = model->meta.head_count;
        bp.ffn.WU = bw->WU;
        bp.ffn.WG = bw->WG;
        bp.ffn.WD = bw->WD;
        bp.ffn.norm_weight = bw->ffn_norm_weight;
        bp.ffn.norm_power = 2.0f;
        bp.ffn.norm_eps = model->meta.layer_norm_rms_epsilon;
        _CHECK(vkllm_llama2_build_transformer_block(context, graph, model->weights.kvcache, hidden, bp, i));
        hidden = graph->nodes->data[graph->nodes->used_n - 1];
    }
    vkllm_tensor *norm_srcs[] = {hidden, model->weights.output_norm_weight};
    vkllm_op_rmsnorm_params np = {2.0f, model->meta.layer_norm_rms_epsilon};
    _CHECK(vkllm_tensor_new(context, "output_norm", hidden->shapes, hidden->dtype, VKLLM_OP_RMSNORM, norm_srcs, 2, &np,
                            sizeof(np), false, &t));
    vkllm_tensor *out_norm = t;
    if (vkllm_graph_add_node(context, graph, out_norm) != VKLLM_ERR_OK)
        return vkllm_tensor_free(context, out_norm), VKLLM_ERR_ALLOC;
    uint32_t logits_shapes[4] = {batch, 1, seq, vocab};
    vkllm_tensor *logit_srcs[] = {out_norm, model->weights.output_weight};
    vkllm_op_matmul_params mm = {1.0f, 0};
    _CHECK(vkllm_tensor_new(context, "logits", logits_shapes, out_norm->dtype, VKLLM_OP_MATMUL, logit_srcs, 2, &mm,
                            sizeof(mm), false, &t));
    vkllm_tensor *logits = t;
    if (vkllm_graph_add_node(context, graph, logits) != VKLLM_ERR_OK)
        return vkllm_tensor_free(context, logits), VKLLM_ERR_ALLOC;
    uint32_t out_shapes[4] = {batch, 1, seq, 1};
    _CHECK(vkllm_tensor_new(context, "output", out_shapes, vkllm_dtype_uint32, VKLLM_OP_ARG_MAX, &logits, 1, nullptr,
                            0, true, &t));
    if (vkllm_graph_add_node(context, graph, t) != VKLLM_ERR_OK)
        return vkllm_tensor_free(context, t), VKLLM_ERR_ALLOC;
    _CHECK(vkllm_graph_set_output(context, graph, t));
    return VKLLM_ERR_OK;
}

extern "C" vkllm_err_t vkllm_models_llama2_build_graph(struct vkllm_context *context, struct vkllm_models_llama2 *model,
                                                       struct vkllm_tensor *input_toks, struct vkllm_graph *graph,
                                                       uint32_t offsets)
{
    DeviceScope device_scope(context);
    _CHECK_ARGS(context && model);
    _CHECK_ARGS(model->weights.tok_embed_weights && model->weights.output_norm_weight &&
                model->weights.output_weight);
    _CHECK_ARGS(model->weights.blocks && model->weights.blocks->used_n > 0);
    _CHECK_ARGS(input_toks && graph);
    vkllm_err_t rc = build_graph_body(context, model, input_toks, graph, offsets);
    if (rc != VKLLM_ERR_OK)
    {
        vkllm_graph_free(context, graph); // src/models/vkllm_models_llama2.c:599-600
        return rc;
    }
    ModelPriv *mp = model_priv(model);
    if (mp && mp->fused_ok && input_toks->shapes[0] == 1 && input_toks->shapes[1] == 1 && input_toks->shapes[2] == 1)
        graph->plan = fused_plan_new(model, input_toks, offsets);
    return VKLLM_ERR_OK;
}

// =============================================================================================================
// tokenizer: src/models/vkllm_models_llama2.c:604-816. Space -> U+2581, a leading U+2581, split into UTF-8
// characters, then repeatedly merge the adjacent pair whose concatenation is the vocabulary entry with the highest
// score (first such pair on ties); pieces outside the vocabulary are dropped; BOS/EOS per metadata.

static int token_id_of(vkllm_models_llama2 *m, const std::string &s)
{
    ModelPriv *mp = model_priv(m);
    if (mp && mp->vocab_index.empty())
        for (size_t i = 0; i < m->meta.tokens->used_n; ++i)
            mp->vocab_index.emplace(m->meta.tokens->data[i].text, (int)i);
    if (mp)
    {
        auto it = mp->vocab_index.find(s);
        return it == mp->vocab_index.end() ? -1 : it->second;
    }
    for (size_t i = 0; i < m->meta.tokens->used_n; ++i)
        if (s == m->meta.tokens->data[i].text)
            return (int)i;
    return -1;
}

extern "C" vkllm_err_t vkllm_models_llama2_tokenize(struct vkllm_models_llama2 *model, const char *sentence,
                                                    struct vkllm_array_token_id **token_ids)
{
    _CHECK_ARGS(model && sentence && token_ids);
    _CHECK_ARGS(model->meta.tokens && model->meta.tokens->used_n > 0);
    const size_t n = strlen(sentence);
    if (n == 0)
        return vkllm_array_token_id_new(token_ids, 1);
    static const char kSpace[] = "\xe2\x96\x81";
    std::string text(kSpace);
    for (size_t i = 0; i < n; ++i)
        if (sentence[i] == ' ')
            text += kSpace;
        else
            text += sentence[i];
    std::vector<std::string> pieces;
    for (size_t i = 0; i < text.size();)
    {
        unsigned char c = (unsigned char)text[i];
        size_t len = 1;
        if (c >= 0x80)
        {
            if ((c & 0xE0) == 0xC0)
                len = 2;
            else if ((c & 0xF0) == 0xE0)
                len = 3;
            else if ((c & 0xF8) == 0xF0)
                len = 4;
        }
        if (i + len > text.size())
            len = text.size() - i;
        pieces.emplace_back(text.substr(i, len));
        i += len;
    }
    while (pieces.size() > 1)
    {
        float best = -INFINITY;
        int best_tok = -1;
        size_t at = 0;
        for (size_t i = 0; i + 1 < pieces.size(); ++i)
        {
            int id = token_id_of(model, pieces[i] + pieces[i + 1]);
            if (id >= 0 && model->meta.tokens->data[id].score > best)
            {
                best = model->meta.tokens->data[id].score;
                best_tok = id;
                at = i;
            }
        }
        if (best_tok < 0)
            break;
        pieces[at] += pieces[at + 1];
        pieces.erase(pieces.begin() + (long)at + 1);
    }
    _CHECK(vkllm_array_token_id_new(token_ids, pieces.size() + 2));
    // a failed append frees the partial list and reports the error: no short id list comes back as a success
    vkllm_err_t err = VKLLM_ERR_OK;
    if (model->meta.add_bos_token)
        err = vkllm_array_token_id_append(*token_ids, model->meta.bos_token_id);
    for (size_t i = 0; i < pieces.size() && err == VKLLM_ERR_OK; ++i)
    {
        int id = token_id_of(model, pieces[i]);
        if (id >= 0)
            err = vkllm_array_token_id_append(*token_ids, (uint32_t)id);
    }
    if (err == VKLLM_ERR_OK && model->meta.add_eos_token)
        err = vkllm_array_token_id_append(*token_ids, model->meta.eos_token_id);
    if (err != VKLLM_ERR_OK)
    {
        log_error("tokenize: appending a token id failed (%s)", vkllm_err_s(err));
        vkllm_array_token_id_free(*token_ids);
        *token_ids = nullptr;
    }
    return err;
}
