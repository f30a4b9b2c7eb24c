/*
 * CPU oracle: LLaMA-2 model (GGUF file, forward step, token loop). TEST INFRASTRUCTURE ONLY -- see oracle.h.
 *
 * The forward step follows the node sequence that vkllm_models_llama2_build_graph creates
 * (src/models/vkllm_models_llama2.c:488-602) with the sub-graphs of src/models/vkllm_llama2_layers.c:13-354 and the
 * KV cache of src/models/vkllm_kvcache.c:65-102. Every node output is rounded to fp16 where the reference stores
 * an fp16 tensor.
 */
#include "oracle.h"

#include <float.h>
#include <math.h>
#include <pthread.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <unistd.h>

/* GGUF v3 constants (public GGUF specification; the reference reads them through antirez/gguf-tools) */
enum
{
    GGUF_T_UINT8 = 0,
    GGUF_T_INT8 = 1,
    GGUF_T_UINT16 = 2,
    GGUF_T_INT16 = 3,
    GGUF_T_UINT32 = 4,
    GGUF_T_INT32 = 5,
    GGUF_T_FLOAT32 = 6,
    GGUF_T_BOOL = 7,
    GGUF_T_STRING = 8,
    GGUF_T_ARRAY = 9,
    GGUF_T_UINT64 = 10,
    GGUF_T_INT64 = 11,
    GGUF_T_FLOAT64 = 12
};
enum
{
    GGML_F32 = 0,
    GGML_F16 = 1
};
#define GGUF_ALIGN 32

struct oracle_model
{
    oracle_llama_cfg cfg;
    uint32_t n_tensors;
    void **tensors;      /* by tensor id (write order); fp16 matrices or f32 norms */
    size_t *counts;      /* elements per tensor */
    uint16_t *kcache;    /* [L][H][ctx][hd] */
    uint16_t *vcache;
    float *freqs;        /* [hd/2] */
};

static float g_h2f[65536];
static pthread_once_t g_h2f_once = PTHREAD_ONCE_INIT;
static void h2f_init(void)
{
    for (uint32_t i = 0; i < 65536; ++i)
        g_h2f[i] = oracle_f16_to_f32((uint16_t)i);
}
static inline float h2f(uint16_t h)
{
    return g_h2f[h];
}

static uint32_t tid_embd(void)
{
    return 0;
}
static uint32_t tid_blk(uint32_t l, uint32_t k)
{
    return 1 + 9 * l + k;
}
enum
{
    K_ATTN_NORM = 0,
    K_Q,
    K_K,
    K_V,
    K_O,
    K_FFN_NORM,
    K_GATE,
    K_UP,
    K_DOWN
};
static uint32_t tid_out_norm(const oracle_llama_cfg *c)
{
    return 1 + 9 * c->n_layer;
}
static uint32_t tid_out(const oracle_llama_cfg *c)
{
    return 2 + 9 * c->n_layer;
}

/* tensor table: name, dims (ne0 = inner), is_norm */
typedef struct
{
    char name[64];
    uint64_t ne0, ne1;
    int ndim;
    int f32;
} tinfo;

static uint32_t make_table(const oracle_llama_cfg *c, tinfo *t)
{
    uint32_t n = 0;
    snprintf(t[n].name, 64, "token_embd.weight");
    t[n].ne0 = c->dim, t[n].ne1 = c->vocab, t[n].ndim = 2, t[n].f32 = 0, n++;
    for (uint32_t l = 0; l < c->n_layer; ++l)
    {
        const char *nm[9] = {"attn_norm", "attn_q",   "attn_k", "attn_v",  "attn_output",
                             "ffn_norm",  "ffn_gate", "ffn_up", "ffn_down"};
        for (int k = 0; k < 9; ++k)
        {
            snprintf(t[n].name, 64, "blk.%u.%s.weight", l, nm[k]);
            t[n].ndim = 2;
            t[n].f32 = 0;
            switch (k)
            {
            case K_ATTN_NORM:
            case K_FFN_NORM:
                t[n].ne0 = c->dim, t[n].ne1 = 1, t[n].ndim = 1, t[n].f32 = 1;
                break;
            case K_Q:
            case K_K:
            case K_V:
            case K_O:
                t[n].ne0 = c->dim, t[n].ne1 = c->dim;
                break;
            case K_GATE:
            case K_UP:
                t[n].ne0 = c->dim, t[n].ne1 = c->ffn;
                break;
            case K_DOWN:
                t[n].ne0 = c->ffn, t[n].ne1 = c->dim;
                break;
            }
            n++;
        }
    }
    snprintf(t[n].name, 64, "output_norm.weight");
    t[n].ne0 = c->dim, t[n].ne1 = 1, t[n].ndim = 1, t[n].f32 = 1, n++;
    snprintf(t[n].name, 64, "output.weight");
    t[n].ne0 = c->dim, t[n].ne1 = c->vocab, t[n].ndim = 2, t[n].f32 = 0, n++;
    return n;
}

/* ------------------------------------------------------------------------------------------------------------ */
/* synthetic tokenizer: <unk>, <s>, </s>, 256 byte tokens, then pieces; score = -id */
static void token_text(uint32_t id, char *buf, size_t n)
{
    static const char *words[] = {"the", "a",  "is",  "of", "and", "to", "in", "what", "largest", "animal",
                                  "Q",   "A",  "whale", "blue", "it", "that", "on", "for", "with", "as"};
    const uint32_t nwords = sizeof(words) / sizeof(words[0]);
    if (id == 0)
        snprintf(buf, n, "<unk>");
    else if (id == 1)
        snprintf(buf, n, "<s>");
    else if (id == 2)
        snprintf(buf, n, "</s>");
    else if (id < 259)
        snprintf(buf, n, "<0x%02X>", id - 3);
    else if (id < 259 + 95)
        snprintf(buf, n, "%c", (char)(32 + (id - 259)));
    else if (id == 259 + 95)
        snprintf(buf, n, "\xe2\x96\x81");
    else if (id < 259 + 96 + nwords)
        snprintf(buf, n, "\xe2\x96\x81%s", words[id - (259 + 96)]);
    else if (id < 259 + 96 + 2 * nwords)
        snprintf(buf, n, "%s", words[id - (259 + 96 + nwords)]);
    else
        snprintf(buf, n, "\xe2\x96\x81tok%u", id);
}

static int token_type(uint32_t id)
{
    if (id == 0)
        return 2;
    if (id < 3)
        return 3;
    if (id < 259)
        return 6;
    return 1;
}

/* ------------------------------------------------------------------------------------------------------------ */
/* GGUF writer */
static void w_u32(FILE *f, uint32_t v)
{
    fwrite(&v, 4, 1, f);
}
static void w_u64(FILE *f, uint64_t v)
{
    fwrite(&v, 8, 1, f);
}
static void w_f32(FILE *f, float v)
{
    fwrite(&v, 4, 1, f);
}
static void w_str(FILE *f, const char *s)
{
    uint64_t n = strlen(s);
    w_u64(f, n);
    fwrite(s, 1, n, f);
}
static void kv_u32(FILE *f, const char *k, uint32_t v)
{
    w_str(f, k);
    w_u32(f, GGUF_T_UINT32);
    w_u32(f, v);
}
static void kv_f32(FILE *f, const char *k, float v)
{
    w_str(f, k);
    w_u32(f, GGUF_T_FLOAT32);
    w_f32(f, v);
}
static void kv_bool(FILE *f, const char *k, int v)
{
    uint8_t b = (uint8_t)(v != 0);
    w_str(f, k);
    w_u32(f, GGUF_T_BOOL);
    fwrite(&b, 1, 1, f);
}
static void kv_str(FILE *f, const char *k, const char *v)
{
    w_str(f, k);
    w_u32(f, GGUF_T_STRING);
    w_str(f, v);
}

typedef struct
{
    const oracle_llama_cfg *cfg;
    uint64_t seed;
    uint32_t id;
    uint16_t *dst;
    size_t begin, end;
} gen_job;

static void *gen_worker(void *p)
{
    gen_job *j = (gen_job *)p;
    uint64_t stream = oracle_tensor_stream(j->seed, j->id);
    for (size_t i = j->begin; i < j->end; ++i)
        j->dst[i - j->begin] = oracle_f32_to_f16(oracle_normal(stream, i) * j->cfg->weight_std);
    return NULL;
}

/* fills dst[0..count) with the weights of tensor `id`, using up to 16 threads for large tensors */
static void gen_weights(const oracle_llama_cfg *cfg, uint64_t seed, uint32_t id, uint16_t *dst, size_t count)
{
    int nt = count > (1u << 22) ? 16 : 1;
    pthread_t th[16];
    gen_job jobs[16];
    size_t chunk = (count + nt - 1) / nt;
    for (int t = 0; t < nt; ++t)
    {
        size_t b = chunk * t, e = b + chunk < count ? b + chunk : count;
        if (b > e)
            b = e;
        jobs[t] = (gen_job){cfg, seed, id, dst + b, b, e};
        if (nt > 1)
            pthread_create(&th[t], NULL, gen_worker, &jobs[t]);
        else
            gen_worker(&jobs[t]);
    }
    if (nt > 1)
        for (int t = 0; t < nt; ++t)
            pthread_join(th[t], NULL);
}

/* ---- parallel loops of the forward step ----
 * fn(arg, i) for i in [0, n), split into contiguous ranges over up to ORACLE_THREADS threads (default: the online
 * CPUs, at most 16) when the loop does enough work. Every index is computed by exactly one thread with the same arithmetic in the same order, so
 * the results do not depend on the thread count. */
typedef void (*par_fn)(void *arg, size_t i);
typedef struct
{
    par_fn fn;
    void *arg;
    size_t begin, end;
} par_job;

static void *par_worker(void *p)
{
    par_job *j = (par_job *)p;
    for (size_t i = j->begin; i < j->end; ++i)
        j->fn(j->arg, i);
    return NULL;
}

static int par_threads(void)
{
    const char *e = getenv("ORACLE_THREADS");
    long n = e && *e ? strtol(e, NULL, 10) : sysconf(_SC_NPROCESSORS_ONLN);
    return n < 1 ? 1 : (n > 16 ? 16 : (int)n);
}

static void par_for(size_t n, par_fn fn, void *arg, double work)
{
    /* thread start-up costs ~20 us: small loops (under ~4M multiply-adds) stay on the calling thread */
    int nt = work < 4e6 ? 1 : par_threads();
    if ((size_t)nt > n)
        nt = (int)n;
    if (nt <= 1)
    {
        for (size_t i = 0; i < n; ++i)
            fn(arg, i);
        return;
    }
    pthread_t th[16];
    par_job jobs[16];
    size_t chunk = (n + nt - 1) / nt;
    for (int t = 0; t < nt; ++t)
    {
        size_t b = chunk * t, e = b + chunk < n ? b + chunk : n;
        jobs[t] = (par_job){fn, arg, b < e ? b : e, e};
        pthread_create(&th[t], NULL, par_worker, &jobs[t]);
    }
    for (int t = 0; t < nt; ++t)
        pthread_join(th[t], NULL);
}

int oracle_gguf_write_random(const char *path, const oracle_llama_cfg *c, uint64_t seed)
{
    FILE *f = fopen(path, "wb");
    if (!f)
        return -1;
    uint32_t nmax = 3 + 9 * c->n_layer;
    tinfo *t = (tinfo *)calloc(nmax, sizeof(tinfo));
    uint32_t nt = make_table(c, t);

    fwrite("GGUF", 1, 4, f);
    w_u32(f, 3);
    w_u64(f, nt);
    w_u64(f, 24);
    kv_str(f, "general.architecture", "llama");
    kv_u32(f, "general.alignment", GGUF_ALIGN);
    kv_u32(f, "llama.block_count", c->n_layer);
    kv_u32(f, "llama.context_length", c->ctx);
    kv_u32(f, "llama.embedding_length", c->dim);
    kv_u32(f, "llama.feed_forward_length", c->ffn);
    kv_u32(f, "llama.attention.head_count", c->n_head);
    kv_u32(f, "llama.attention.head_count_kv", c->n_head_kv);
    kv_f32(f, "llama.attention.layer_norm_rms_epsilon", c->eps);
    kv_f32(f, "llama.rope.freq_base", c->theta);
    kv_u32(f, "llama.attention.key_length", c->dim / c->n_head);
    kv_u32(f, "llama.attention.value_length", c->dim / c->n_head);
    kv_u32(f, "llama.vocab_size", c->vocab);
    kv_str(f, "tokenizer.ggml.model", "llama");
    /* tokens */
    w_str(f, "tokenizer.ggml.tokens");
    w_u32(f, GGUF_T_ARRAY);
    w_u32(f, GGUF_T_STRING);
    w_u64(f, c->vocab);
    char buf[64];
    for (uint32_t i = 0; i < c->vocab; ++i)
    {
        token_text(i, buf, sizeof(buf));
        w_str(f, buf);
    }
    w_str(f, "tokenizer.ggml.scores");
    w_u32(f, GGUF_T_ARRAY);
    w_u32(f, GGUF_T_FLOAT32);
    w_u64(f, c->vocab);
    for (uint32_t i = 0; i < c->vocab; ++i)
        w_f32(f, -(float)i);
    w_str(f, "tokenizer.ggml.token_type");
    w_u32(f, GGUF_T_ARRAY);
    w_u32(f, GGUF_T_INT32);
    w_u64(f, c->vocab);
    for (uint32_t i = 0; i < c->vocab; ++i)
    {
        int32_t ty = token_type(i);
        fwrite(&ty, 4, 1, f);
    }
    kv_u32(f, "tokenizer.ggml.bos_token_id", c->bos_id);
    kv_u32(f, "tokenizer.ggml.eos_token_id", c->eos_id);
    kv_u32(f, "tokenizer.ggml.padding_token_id", c->pad_id);
    kv_bool(f, "tokenizer.ggml.add_bos_token", 1);
    kv_bool(f, "tokenizer.ggml.add_eos_token", 0);
    kv_u32(f, "general.file_type", 1);
    kv_str(f, "general.name", "vkllm-random-llama2");

    uint64_t off = 0;
    for (uint32_t i = 0; i < nt; ++i)
    {
        w_str(f, t[i].name);
        w_u32(f, (uint32_t)t[i].ndim);
        w_u64(f, t[i].ne0);
        if (t[i].ndim == 2)
            w_u64(f, t[i].ne1);
        w_u32(f, t[i].f32 ? GGML_F32 : GGML_F16);
        w_u64(f, off);
        uint64_t bytes = t[i].ne0 * t[i].ne1 * (t[i].f32 ? 4 : 2);
        off += (bytes + GGUF_ALIGN - 1) / GGUF_ALIGN * GGUF_ALIGN;
    }
    long pos = ftell(f);
    long pad = (GGUF_ALIGN - pos % GGUF_ALIGN) % GGUF_ALIGN;
    static const char zeros[GGUF_ALIGN] = {0};
    fwrite(zeros, 1, (size_t)pad, f);

    for (uint32_t i = 0; i < nt; ++i)
    {
        size_t count = (size_t)(t[i].ne0 * t[i].ne1);
        uint64_t bytes = count * (t[i].f32 ? 4 : 2);
        if (t[i].f32)
        {
            float *v = (float *)malloc(bytes);
            for (size_t k = 0; k < count; ++k)
                v[k] = 1.0f;
            fwrite(v, 1, bytes, f);
            free(v);
        }
        else
        {
            uint16_t *v = (uint16_t *)malloc(bytes);
            gen_weights(c, seed, i, v, count);
            fwrite(v, 1, bytes, f);
            free(v);
        }
        uint64_t padded = (bytes + GGUF_ALIGN - 1) / GGUF_ALIGN * GGUF_ALIGN;
        fwrite(zeros, 1, (size_t)(padded - bytes), f);
    }
    free(t);
    return fclose(f) == 0 ? 0 : -1;
}

/* ------------------------------------------------------------------------------------------------------------ */
/* GGUF reader */
typedef struct
{
    const uint8_t *p, *end;
    int err;
} rdr;

static uint64_t r_n(rdr *r, size_t n)
{
    uint64_t v = 0;
    if ((size_t)(r->end - r->p) < n)
    {
        r->err = 1;
        return 0;
    }
    memcpy(&v, r->p, n);
    r->p += n;
    return v;
}
static float r_f32(rdr *r)
{
    uint32_t v = (uint32_t)r_n(r, 4);
    float f;
    memcpy(&f, &v, 4);
    return f;
}
static const char *r_str(rdr *r, uint64_t *len)
{
    *len = r_n(r, 8);
    if (r->err || (uint64_t)(r->end - r->p) < *len)
    {
        r->err = 1;
        return "";
    }
    const char *s = (const char *)r->p;
    r->p += *len;
    return s;
}
static size_t scalar_size(uint32_t ty)
{
    switch (ty)
    {
    case GGUF_T_UINT8:
    case GGUF_T_INT8:
    case GGUF_T_BOOL:
        return 1;
    case GGUF_T_UINT16:
    case GGUF_T_INT16:
        return 2;
    case GGUF_T_UINT32:
    case GGUF_T_INT32:
    case GGUF_T_FLOAT32:
        return 4;
    case GGUF_T_UINT64:
    case GGUF_T_INT64:
    case GGUF_T_FLOAT64:
        return 8;
    }
    return 0;
}
static void skip_value(rdr *r, uint32_t ty)
{
    if (ty == GGUF_T_STRING)
    {
        uint64_t n;
        r_str(r, &n);
    }
    else if (ty == GGUF_T_ARRAY)
    {
        uint32_t et = (uint32_t)r_n(r, 4);
        uint64_t cnt = r_n(r, 8);
        for (uint64_t i = 0; i < cnt && !r->err; ++i)
            skip_value(r, et);
    }
    else
    {
        size_t s = scalar_size(ty);
        if (!s)
            r->err = 1;
        else
            r->p += s;
    }
}
static int key_is(const char *k, uint64_t n, const char *lit)
{
    return strlen(lit) == n && memcmp(k, lit, n) == 0;
}

static oracle_model *model_alloc(const oracle_llama_cfg *c)
{
    pthread_once(&g_h2f_once, h2f_init);
    oracle_model *m = (oracle_model *)calloc(1, sizeof(*m));
    m->cfg = *c;
    m->n_tensors = 3 + 9 * c->n_layer;
    m->tensors = (void **)calloc(m->n_tensors, sizeof(void *));
    m->counts = (size_t *)calloc(m->n_tensors, sizeof(size_t));
    uint32_t hd = c->dim / c->n_head;
    size_t cache = (size_t)c->n_layer * c->n_head * c->ctx * hd;
    m->kcache = (uint16_t *)calloc(cache, 2);
    m->vcache = (uint16_t *)calloc(cache, 2);
    m->freqs = (float *)malloc(sizeof(float) * (hd / 2 + 1));
    oracle_rope_freqs(c->theta, hd, m->freqs);
    return m;
}

oracle_model *oracle_model_load(const char *path)
{
    FILE *f = fopen(path, "rb");
    if (!f)
        return NULL;
    fseek(f, 0, SEEK_END);
    long sz = ftell(f);
    fseek(f, 0, SEEK_SET);
    uint8_t *buf = (uint8_t *)malloc((size_t)sz);
    if (!buf || fread(buf, 1, (size_t)sz, f) != (size_t)sz)
    {
        fclose(f);
        free(buf);
        return NULL;
    }
    fclose(f);
    rdr r = {buf, buf + sz, 0};
    if (memcmp(buf, "GGUF", 4) != 0)
    {
        free(buf);
        return NULL;
    }
    r.p += 4;
    uint32_t version = (uint32_t)r_n(&r, 4);
    uint64_t nt = r_n(&r, 8), nkv = r_n(&r, 8);
    if (version != 3)
    {
        free(buf);
        return NULL;
    }
    /* defaults of src/models/vkllm_models_llama2.c:224-241 */
    oracle_llama_cfg c = {32, 4096, 32, 32, 11008, 32000, 2048, 1e-6f, 10000.0f, 1, 2, 0, 0.02f};
    uint32_t align = GGUF_ALIGN;
    for (uint64_t i = 0; i < nkv && !r.err; ++i)
    {
        uint64_t kl;
        const char *k = r_str(&r, &kl);
        uint32_t ty = (uint32_t)r_n(&r, 4);
        if (ty == GGUF_T_UINT32 || ty == GGUF_T_FLOAT32)
        {
            const uint8_t *save = r.p;
            uint32_t u = (uint32_t)r_n(&r, 4);
            r.p = save;
            float fv = r_f32(&r);
            if (ty == GGUF_T_UINT32)
            {
                if (key_is(k, kl, "llama.block_count"))
                    c.n_layer = u;
                else if (key_is(k, kl, "llama.context_length"))
                    c.ctx = u;
                else if (key_is(k, kl, "llama.embedding_length"))
                    c.dim = u;
                else if (key_is(k, kl, "llama.feed_forward_length"))
                    c.ffn = u;
                else if (key_is(k, kl, "llama.attention.head_count"))
                    c.n_head = u;
                else if (key_is(k, kl, "llama.attention.head_count_kv"))
                    c.n_head_kv = u;
                else if (key_is(k, kl, "llama.vocab_size"))
                    c.vocab = u;
                else if (key_is(k, kl, "tokenizer.ggml.bos_token_id"))
                    c.bos_id = u;
                else if (key_is(k, kl, "tokenizer.ggml.eos_token_id"))
                    c.eos_id = u;
                else if (key_is(k, kl, "tokenizer.ggml.padding_token_id"))
                    c.pad_id = u;
                else if (key_is(k, kl, "general.alignment"))
                    align = u;
            }
            else
            {
                if (key_is(k, kl, "llama.attention.layer_norm_rms_epsilon"))
                    c.eps = fv;
                else if (key_is(k, kl, "llama.rope.freq_base"))
                    c.theta = fv;
            }
        }
        else
            skip_value(&r, ty);
    }
    if (r.err)
    {
        free(buf);
        return NULL;
    }
    typedef struct
    {
        char name[96];
        uint64_t ne[4];
        uint32_t ndim, type;
        uint64_t off;
    } ti;
    ti *infos = (ti *)calloc(nt, sizeof(ti));
    for (uint64_t i = 0; i < nt && !r.err; ++i)
    {
        uint64_t nl;
        const char *nm = r_str(&r, &nl);
        size_t cp = nl < 95 ? nl : 95;
        memcpy(infos[i].name, nm, cp);
        infos[i].ndim = (uint32_t)r_n(&r, 4);
        for (uint32_t d = 0; d < 4; ++d)
            infos[i].ne[d] = 1;
        for (uint32_t d = 0; d < infos[i].ndim && d < 4; ++d)
            infos[i].ne[d] = r_n(&r, 8);
        infos[i].type = (uint32_t)r_n(&r, 4);
        infos[i].off = r_n(&r, 8);
    }
    size_t data_start = (size_t)(r.p - buf);
    data_start = (data_start + align - 1) / align * align;
    oracle_model *m = model_alloc(&c);
    /* vocab may be absent from the keys: take it from token_embd */
    for (uint64_t i = 0; i < nt; ++i)
    {
        int id = -1;
        unsigned l;
        char rest[64];
        if (strcmp(infos[i].name, "token_embd.weight") == 0)
            id = (int)tid_embd();
        else if (strcmp(infos[i].name, "output_norm.weight") == 0)
            id = (int)tid_out_norm(&c);
        else if (strcmp(infos[i].name, "output.weight") == 0)
            id = (int)tid_out(&c);
        else if (sscanf(infos[i].name, "blk.%u.%63s", &l, rest) == 2 && l < c.n_layer)
        {
            const char *nm[9] = {"attn_norm.weight", "attn_q.weight",   "attn_k.weight",
                                 "attn_v.weight",    "attn_output.weight", "ffn_norm.weight",
                                 "ffn_gate.weight",  "ffn_up.weight",   "ffn_down.weight"};
            for (int k = 0; k < 9; ++k)
                if (strcmp(rest, nm[k]) == 0)
                    id = (int)tid_blk(l, (uint32_t)k);
        }
        if (id < 0)
            continue;
        size_t count = (size_t)(infos[i].ne[0] * infos[i].ne[1] * infos[i].ne[2] * infos[i].ne[3]);
        size_t es = infos[i].type == GGML_F32 ? 4 : 2;
        const uint8_t *src = buf + data_start + infos[i].off;
        if (src + count * es > buf + sz)
            continue;
        void *dst = malloc(count * es);
        memcpy(dst, src, count * es);
        m->tensors[id] = dst;
        m->counts[id] = count;
        if (id == (int)tid_embd())
            m->cfg.vocab = (uint32_t)infos[i].ne[1];
    }
    free(infos);
    free(buf);
    for (uint32_t i = 0; i < m->n_tensors; ++i)
        if (!m->tensors[i])
        {
            oracle_model_free(m);
            return NULL;
        }
    return m;
}

oracle_model *oracle_model_random(const oracle_llama_cfg *c, uint64_t seed)
{
    oracle_model *m = model_alloc(c);
    uint32_t nmax = 3 + 9 * c->n_layer;
    tinfo *t = (tinfo *)calloc(nmax, sizeof(tinfo));
    uint32_t nt = make_table(c, t);
    for (uint32_t i = 0; i < nt; ++i)
    {
        size_t count = (size_t)(t[i].ne0 * t[i].ne1);
        if (t[i].f32)
        {
            float *v = (float *)malloc(count * 4);
            for (size_t k = 0; k < count; ++k)
                v[k] = 1.0f;
            m->tensors[i] = v;
        }
        else
        {
            uint16_t *v = (uint16_t *)malloc(count * 2);
            gen_weights(c, seed, i, v, count);
            m->tensors[i] = v;
        }
        m->counts[i] = count;
    }
    free(t);
    return m;
}

void oracle_model_free(oracle_model *m)
{
    if (!m)
        return;
    for (uint32_t i = 0; i < m->n_tensors; ++i)
        free(m->tensors[i]);
    free(m->tensors);
    free(m->counts);
    free(m->kcache);
    free(m->vcache);
    free(m->freqs);
    free(m);
}

int oracle_model_cfg(const oracle_model *m, oracle_llama_cfg *cfg)
{
    *cfg = m->cfg;
    return 0;
}

const uint16_t *oracle_model_weight(const oracle_model *m, uint32_t id, size_t *count)
{
    if (id >= m->n_tensors)
        return NULL;
    if (count)
        *count = m->counts[id];
    return (const uint16_t *)m->tensors[id];
}

/* ------------------------------------------------------------------------------------------------------------ */
/* REF16: fp16 arithmetic of the reference's f16f16 shader variants (declared with their citations in oracle.h) */

static int g_ref16 = 0;
static uint32_t g_sub = 8;

void oracle_set_numerics(int ref16, uint32_t subgroup)
{
    g_ref16 = ref16 != 0;
    g_sub = subgroup ? subgroup : 8;
}

/* the fp32 mode's summation order (oracle.h): 0 double sums, 1 sequential fp32 sums */
static int g_acc32 = 0;

void oracle_set_accumulation(int fp32_sequential)
{
    g_acc32 = fp32_sequential != 0;
}

uint16_t oracle_f64_to_f16(double d)
{
    uint64_t x;
    memcpy(&x, &d, 8);
    const uint16_t sign = (uint16_t)((x >> 48) & 0x8000u);
    const int exp = (int)((x >> 52) & 0x7ffu);
    const uint64_t mant = x & 0xfffffffffffffull;
    if (exp == 0x7ff)
        return (uint16_t)(sign | (mant ? 0x7e00u : 0x7c00u));
    if (exp == 0) /* zero, or a double subnormal: far below half the smallest fp16 subnormal */
        return sign;
    const int e = exp - 1023;
    if (e > 15)
        return (uint16_t)(sign | 0x7c00u);
    if (e < -25) /* below half of 2^-24 */
        return sign;
    const uint64_t full = mant | (1ull << 52); /* value = full * 2^(e - 52) */
    /* kept bits: 11 for a normal result (exponent >= -14), fewer for a subnormal one (units of 2^-24) */
    const int shift = e >= -14 ? 42 : 42 + (-14 - e);
    uint64_t m = full >> shift;
    const uint64_t rem = full & ((1ull << shift) - 1), half = 1ull << (shift - 1);
    if (rem > half || (rem == half && (m & 1u)))
        ++m;
    if (e < -14) /* subnormal; a carry into 0x400 is the smallest normal, the same bits */
        return (uint16_t)(sign | (uint16_t)m);
    uint32_t hexp = (uint32_t)(e + 15);
    if (m == 0x800u)
    {
        m = 0x400u;
        ++hexp;
    }
    if (hexp >= 31)
        return (uint16_t)(sign | 0x7c00u);
    return (uint16_t)(sign | (hexp << 10) | (uint32_t)(m & 0x3ffu));
}

/* the exact result of one fp16 operation, rounded to fp16 and read back */
static inline float r16(double v)
{
    return h2f(oracle_f64_to_f16(v));
}

/* exp, cos, sin and pow of fp16 arguments as correctly rounded fp16 values */
static inline float exp16(float v)
{
    return r16(exp((double)v));
}

static float gemv16_value(const uint16_t *x, const uint16_t *w, uint32_t K, float scale, int act, uint32_t G)
{
    float total = 0.f;
    for (uint32_t l = 0; l < G; ++l)
    {
        /* lane l: fp16 accumulator += fp16(dot(vec4 a, vec4 b) in fp32) for i = 4l, 4l + 4G, ... */
        float acc = 0.f;
        for (uint32_t i = 4 * l; i + 3 < K; i += 4 * G)
        {
            float d = h2f(x[i]) * h2f(w[i]);
            d = d + h2f(x[i + 1]) * h2f(w[i + 1]);
            d = d + h2f(x[i + 2]) * h2f(w[i + 2]);
            d = d + h2f(x[i + 3]) * h2f(w[i + 3]);
            acc = r16((double)r16(d) + acc);
        }
        /* subgroupAdd in fp16, lanes in order */
        total = l == 0 ? acc : r16((double)total + acc);
    }
    float v = r16((double)total * r16(scale));
    if (act) /* v / (1 + exp(-v)) in fp16 */
        v = r16((double)v / r16(1.0 + exp16(r16(-(double)v))));
    return v;
}

uint16_t oracle_gemv16(const uint16_t *x, const uint16_t *w, uint32_t K, float scale, int act, uint32_t subgroup)
{
    pthread_once(&g_h2f_once, h2f_init);
    return oracle_f32_to_f16(gemv16_value(x, w, K, scale, act, subgroup ? subgroup : 8));
}

/* fp16 dot(f16vec2) of pairs read with element strides sa, sb, accumulated in fp32 */
static float gemm16_dot_strided(const uint16_t *a, size_t sa, const uint16_t *b, size_t sb, uint32_t K)
{
    float acc = 0.f;
    for (uint32_t k = 0; k < K; k += 2)
    {
        const float p0 = r16((double)h2f(a[k * sa]) * h2f(b[k * sb]));
        const float p1 = k + 1 < K ? r16((double)h2f(a[(k + 1) * sa]) * h2f(b[(k + 1) * sb])) : 0.f;
        acc += r16((double)p0 + p1);
    }
    return acc;
}

float oracle_gemm16_dot(const uint16_t *a, const uint16_t *b, uint32_t K)
{
    pthread_once(&g_h2f_once, h2f_init);
    return gemm16_dot_strided(a, 1, b, 1, K);
}

void oracle_softmax16_row(const uint16_t *x, uint16_t *out, uint32_t W, uint32_t limit, uint32_t subgroup)
{
    pthread_once(&g_h2f_once, h2f_init);
    const uint32_t G = subgroup ? subgroup : 8;
    float mx = h2f(x[0]); /* the max over the whole row, masked entries included: exact in any precision */
    for (uint32_t i = 0; i < W; ++i)
        mx = h2f(x[i]) > mx ? h2f(x[i]) : mx;
    float total = 0.f;
    for (uint32_t l = 0; l < G; ++l)
    {
        float acc = 0.f;
        for (uint32_t i = l; i < W; i += G)
            if (i <= limit)
                acc = r16((double)acc + exp16(r16((double)h2f(x[i]) - mx)));
        total = l == 0 ? acc : r16((double)total + acc);
    }
    for (uint32_t i = 0; i < W; ++i)
        out[i] = i > limit ? 0 : oracle_f64_to_f16((double)exp16(r16((double)h2f(x[i]) - mx)) / total);
}

void oracle_rope16_pair(uint16_t v0, uint16_t v1, uint32_t pos, uint32_t w, uint32_t hd, float base, uint16_t *o0,
                        uint16_t *o1)
{
    pthread_once(&g_h2f_once, h2f_init);
    /* f = fp16(pos) / pow(fp16(base), fp16(2w) / fp16(hd)), each operation in fp16 */
    const float e = r16((double)r16(2.0 * w) / r16((double)hd));
    const float pw = r16(pow((double)r16((double)base), (double)e));
    const float f = r16((double)r16((double)pos) / pw);
    const float c = r16(cos((double)f)), sn = r16(sin((double)f));
    const float a = h2f(v0), b = h2f(v1);
    *o0 = oracle_f64_to_f16((double)r16((double)c * a) - r16((double)sn * b));
    *o1 = oracle_f64_to_f16((double)r16((double)sn * a) + r16((double)c * b));
}

/* ------------------------------------------------------------------------------------------------------------ */
/* forward step */

/* y[s][n] = fp16(act(scale * sum_k x[s][k] W[n][k])): VKLLM_OP_MATMUL with a [N,K] weight
 * (src/shaders/vkllm_mat_mul_vec.comp:94-150 for S == 1, src/shaders/vkllm_matmul_t1.comp:156-250 otherwise) */
typedef struct
{
    const double *xd;
    const uint16_t *x16;
    const uint16_t *W;
    uint16_t *y;
    uint32_t S, K, N;
    int act;
} linear_job;

static void linear_row(void *p, size_t n)
{
    const linear_job *j = (const linear_job *)p;
    const uint32_t K = j->K;
    const uint16_t *w = j->W + n * K;
    if (g_ref16)
    {
        /* one token: mat_mul_vec f16f16; more: the tiled GEMM f16f16f16 (fp16 pair dots, fp32 sum and epilogue) */
        for (uint32_t s = 0; s < j->S; ++s)
        {
            const uint16_t *xs = j->x16 + (size_t)s * K;
            float v;
            if (j->S == 1)
                v = gemv16_value(xs, w, K, 1.0f, j->act, g_sub);
            else
            {
                v = oracle_gemm16_dot(xs, w, K) * 1.0f;
                if (j->act)
                    v = v / (1.0f + expf(-v));
            }
            j->y[(size_t)s * j->N + n] = oracle_f32_to_f16(v);
        }
        return;
    }
    /* The weight row is converted once, then TB tokens at a time: every output keeps its own sum, added in k order
     * exactly as for one token alone (the tokens' independent chains only overlap in time). */
    enum
    {
        TB = 8
    };
    double wd[K];
    float wf[K];
    if (j->S >= TB) /* a single token reads the row directly (one pass over the weights) */
        for (uint32_t k = 0; k < K; ++k)
        {
            wf[k] = h2f(w[k]);
            wd[k] = wf[k];
        }
    for (uint32_t s0 = 0; s0 < j->S;)
    {
        /* TB tokens at once while that many remain, then one at a time */
        const uint32_t nb = j->S - s0 >= TB ? TB : 1;
        float v[TB];
        if (nb == TB)
        {
            const double *xs[TB];
            for (uint32_t t = 0; t < TB; ++t)
                xs[t] = j->xd + (size_t)(s0 + t) * K;
            if (g_acc32)
            {
                /* fp16 x fp16 products are exact in fp32; each addition rounds */
                float acc[TB] = {0};
                for (uint32_t k = 0; k < K; ++k)
                    for (uint32_t t = 0; t < TB; ++t)
                        acc[t] += (float)xs[t][k] * wf[k];
                for (uint32_t t = 0; t < TB; ++t)
                    v[t] = acc[t] * 1.0f;
            }
            else
            {
                double acc[TB] = {0};
                for (uint32_t k = 0; k < K; ++k)
                    for (uint32_t t = 0; t < TB; ++t)
                        acc[t] += xs[t][k] * wd[k];
                for (uint32_t t = 0; t < TB; ++t)
                    v[t] = (float)acc[t] * 1.0f;
            }
        }
        else
        {
            const double *xs = j->xd + (size_t)s0 * K;
            if (g_acc32)
            {
                float acc = 0.f;
                for (uint32_t k = 0; k < K; ++k)
                    acc += (float)xs[k] * h2f(w[k]);
                v[0] = acc * 1.0f;
            }
            else
            {
                double acc = 0.0;
                for (uint32_t k = 0; k < K; ++k)
                    acc += xs[k] * (double)h2f(w[k]);
                v[0] = (float)acc * 1.0f;
            }
        }
        for (uint32_t t = 0; t < nb; ++t)
        {
            float y = v[t];
            if (j->act)
                y = y / (1.0f + expf(-y));
            j->y[(size_t)(s0 + t) * j->N + n] = oracle_f32_to_f16(y);
        }
        s0 += nb;
    }
}

static void linear(const uint16_t *x, const uint16_t *W, uint16_t *y, uint32_t S, uint32_t K, uint32_t N, int act)
{
    double *xd = (double *)malloc(sizeof(double) * K * S);
    for (size_t i = 0; i < (size_t)K * S; ++i)
        xd[i] = h2f(x[i]);
    linear_job j = {xd, x, W, y, S, K, N, act};
    par_for(N, linear_row, &j, (double)N * S * K);
    free(xd);
}

/* src/shaders/vkllm_rmsnorm.comp:31-82 over S contiguous rows */
static void rmsnorm_rows(const uint16_t *x, const float *w, uint16_t *y, uint32_t S, uint32_t D, float eps)
{
    for (uint32_t s = 0; s < S; ++s)
    {
        const uint16_t *xr = x + (size_t)s * D;
        double ss = 0.0;
        float ss32 = 0.f;
        for (uint32_t i = 0; i < D; ++i)
        {
            double v = h2f(xr[i]);
            ss += v * v;
            ss32 += (float)v * (float)v;
        }
        float mean = (g_acc32 ? ss32 : (float)ss) / (float)D;
        float alpha = 1.0f / sqrtf(mean + eps);
        for (uint32_t i = 0; i < D; ++i)
            y[(size_t)s * D + i] = oracle_f32_to_f16((h2f(xr[i]) * w[i]) * alpha);
    }
}

static void add_rows(uint16_t *h, const uint16_t *o, size_t n)
{
    for (size_t i = 0; i < n; ++i)
        h[i] = oracle_f32_to_f16(h2f(h[i]) + h2f(o[i]));
}

/* One attention row: head hh, query row s of the step (src/models/vkllm_llama2_layers.c:223-281). */
typedef struct
{
    const uint16_t *rq; /* [H][S][hd] rotated queries */
    const uint16_t *kc, *vc; /* the layer's caches [H][ctx][hd] */
    uint16_t *att; /* [S][D] */
    uint32_t S, offset, kv, D, hd, ctx;
    float scale;
} attn_job;

static void attn_row(void *p, size_t i)
{
    const attn_job *a = (const attn_job *)p;
    const uint32_t S = a->S, offset = a->offset, kv = a->kv, D = a->D, hd = a->hd, ctx = a->ctx;
    const uint32_t hh = (uint32_t)(i / S), s = (uint32_t)(i % S);
    const uint16_t *kc = a->kc, *vc = a->vc;
    uint16_t *att = a->att;
    const float scale = a->scale;
    uint16_t *sc = (uint16_t *)malloc((size_t)kv * 2);
    uint16_t *pr = (uint16_t *)malloc((size_t)kv * 2);
    const uint16_t *qr = a->rq + ((size_t)hh * S + s) * hd;

    if (g_ref16)
    {
        /* scores: mat_mul_vec f16f16 for one query row, else the tiled GEMM (fp32 scale in its epilogue) */
        for (uint32_t j = 0; j < kv; ++j)
        {
            const uint16_t *kr = kc + ((size_t)hh * ctx + j) * hd;
            sc[j] = S == 1 ? oracle_gemv16(qr, kr, hd, scale, 0, g_sub)
                           : oracle_f32_to_f16(oracle_gemm16_dot(qr, kr, hd) * scale);
        }
        oracle_softmax16_row(sc, pr, kv, s + offset, g_sub);
        /* attn . V: the tiled GEMM over key pairs (V read [kv, hd]); when kv == hd, is_transposed_b reads V as
         * [N, K] and one query row takes mat_mul_vec */
        const int tr = kv == hd;
        for (uint32_t n = 0; n < hd; ++n)
        {
            float v;
            if (tr && S == 1)
                v = gemv16_value(pr, vc + ((size_t)hh * ctx + n) * hd, kv, 1.0f, 0, g_sub);
            else if (tr)
                v = gemm16_dot_strided(pr, 1, vc + ((size_t)hh * ctx + n) * hd, 1, kv);
            else
                v = gemm16_dot_strided(pr, 1, vc + (size_t)hh * ctx * hd + n, hd, kv);
            att[(size_t)s * D + (size_t)hh * hd + n] = oracle_f32_to_f16(v * 1.0f);
        }
        free(sc);
        free(pr);
        return;
    }

    /* scores = fp16(scale * q.k) (src/models/vkllm_llama2_layers.c:223-233). Four keys at a time: each score keeps
     * its own sum over d in order (the keys' independent chains only overlap in time). */
    float qf[hd];
    for (uint32_t d = 0; d < hd; ++d)
        qf[d] = h2f(qr[d]);
    uint32_t j0 = 0;
    for (; j0 + 4 <= kv; j0 += 4)
    {
        const uint16_t *kr[4];
        for (int t = 0; t < 4; ++t)
            kr[t] = kc + ((size_t)hh * ctx + j0 + t) * hd;
        if (g_acc32)
        {
            float acc[4] = {0};
            for (uint32_t d = 0; d < hd; ++d)
                for (int t = 0; t < 4; ++t)
                    acc[t] += qf[d] * h2f(kr[t][d]);
            for (int t = 0; t < 4; ++t)
                sc[j0 + t] = oracle_f32_to_f16(acc[t] * scale);
        }
        else
        {
            double acc[4] = {0};
            for (uint32_t d = 0; d < hd; ++d)
                for (int t = 0; t < 4; ++t)
                    acc[t] += (double)qf[d] * (double)h2f(kr[t][d]);
            for (int t = 0; t < 4; ++t)
                sc[j0 + t] = oracle_f32_to_f16((float)acc[t] * scale);
        }
    }
    for (uint32_t j = j0; j < kv; ++j)
    {
        const uint16_t *kr = kc + ((size_t)hh * ctx + j) * hd;
        double acc = 0.0;
        float acc32 = 0.f;
        for (uint32_t d = 0; d < hd; ++d)
        {
            acc += (double)qf[d] * (double)h2f(kr[d]);
            acc32 += qf[d] * h2f(kr[d]);
        }
        sc[j] = oracle_f32_to_f16((g_acc32 ? acc32 : (float)acc) * scale);
    }
    /* SOFTMAX seq_mask=1, offsets=offset (layers.c:237-245, softmax.comp:53-95) */
    float mx = h2f(sc[0]);
    for (uint32_t j = 0; j < kv; ++j)
        mx = h2f(sc[j]) > mx ? h2f(sc[j]) : mx;
    double sum = 0.0;
    float sum32 = 0.f;
    for (uint32_t j = 0; j <= s + offset && j < kv; ++j)
    {
        sum += expf(h2f(sc[j]) - mx);
        sum32 += expf(h2f(sc[j]) - mx);
    }
    float sf = g_acc32 ? sum32 : (float)sum;
    for (uint32_t j = 0; j < kv; ++j)
        pr[j] = j > s + offset ? 0 : oracle_f32_to_f16(expf(h2f(sc[j]) - mx) / sf);
    /* attn . V (layers.c:247-257). When kv == hd, is_transposed_b (src/core/vkllm_op_matmul.c:14-24)
     * reads the [kv, hd] V slice as [N, K] and the product becomes attn . V^T. Eight outputs at a time, each summed
     * over j in order. */
    int transposed = (kv == hd);
    const uint16_t *vh = vc + (size_t)hh * ctx * hd;
    for (uint32_t n0 = 0; n0 < hd; n0 += 8)
    {
        const uint32_t nb = hd - n0 < 8 ? hd - n0 : 8;
        double acc[8] = {0};
        float acc32[8] = {0};
        for (uint32_t j = 0; j < kv; ++j)
        {
            const float p = h2f(pr[j]);
            for (uint32_t t = 0; t < nb; ++t)
            {
                const uint16_t vv = transposed ? vh[(size_t)(n0 + t) * hd + j] : vh[(size_t)j * hd + n0 + t];
                if (g_acc32)
                    acc32[t] += p * h2f(vv);
                else
                    acc[t] += (double)p * (double)h2f(vv);
            }
        }
        /* permute + COPY into [S, H*hd] (layers.c:259-281) */
        for (uint32_t t = 0; t < nb; ++t)
            att[(size_t)s * D + (size_t)hh * hd + n0 + t] =
                oracle_f32_to_f16((g_acc32 ? acc32[t] : (float)acc[t]) * 1.0f);
    }

    free(sc);
    free(pr);
}

int oracle_model_step(oracle_model *m, const uint32_t *toks, uint32_t S, uint32_t offset, uint32_t *out_ids,
                      uint16_t *logits_out, uint16_t *hidden_out)
{
    const oracle_llama_cfg *c = &m->cfg;
    const uint32_t D = c->dim, H = c->n_head, hd = D / H, F = c->ffn, V = c->vocab, ctx = c->ctx;
    if (S == 0 || offset + S > ctx)
        return -1;
    const uint32_t kv = offset + S;
    const float scale = 1.0f / sqrtf((float)hd); /* src/models/vkllm_llama2_layers.c:228 */

    uint16_t *h = (uint16_t *)malloc((size_t)S * D * 2);
    uint16_t *xn = (uint16_t *)malloc((size_t)S * D * 2);
    uint16_t *q = (uint16_t *)malloc((size_t)S * D * 2);
    uint16_t *k = (uint16_t *)malloc((size_t)S * D * 2);
    uint16_t *v = (uint16_t *)malloc((size_t)S * D * 2);
    uint16_t *rq = (uint16_t *)malloc((size_t)S * D * 2); /* [H][S][hd] */
    uint16_t *att = (uint16_t *)malloc((size_t)S * D * 2);
    uint16_t *o = (uint16_t *)malloc((size_t)S * D * 2);
    uint16_t *up = (uint16_t *)malloc((size_t)S * F * 2);
    uint16_t *gate = (uint16_t *)malloc((size_t)S * F * 2);
    uint16_t *logits = (uint16_t *)malloc((size_t)S * V * 2);

    /* EMBEDDING with unk = padding_token_id (src/models/vkllm_models_llama2.c:505-513) */
    const uint16_t *embd = (const uint16_t *)m->tensors[tid_embd()];
    for (uint32_t s = 0; s < S; ++s)
    {
        uint32_t t = toks[s] < V ? toks[s] : c->pad_id;
        memcpy(h + (size_t)s * D, embd + (size_t)t * D, (size_t)D * 2);
    }

    for (uint32_t l = 0; l < c->n_layer; ++l)
    {
        const float *an = (const float *)m->tensors[tid_blk(l, K_ATTN_NORM)];
        const float *fn = (const float *)m->tensors[tid_blk(l, K_FFN_NORM)];
        uint16_t *kc = m->kcache + (size_t)l * H * ctx * hd;
        uint16_t *vc = m->vcache + (size_t)l * H * ctx * hd;

        /* attention sub-graph, src/models/vkllm_llama2_layers.c:133-301 */
        rmsnorm_rows(h, an, xn, S, D, c->eps);
        linear(xn, (const uint16_t *)m->tensors[tid_blk(l, K_Q)], q, S, D, D, 0);
        linear(xn, (const uint16_t *)m->tensors[tid_blk(l, K_K)], k, S, D, D, 0);
        linear(xn, (const uint16_t *)m->tensors[tid_blk(l, K_V)], v, S, D, D, 0);
        /* views [S,D] -> [S,H,hd] -> [H,S,hd]; RoPE (normal style) at position offset + s (rope.comp:39-79);
         * KV append (update_rows) at row offset + s */
        for (uint32_t hh = 0; hh < H; ++hh)
            for (uint32_t s = 0; s < S; ++s)
                for (uint32_t w = 0; w < hd / 2; ++w)
                {
                    size_t src = (size_t)s * D + (size_t)hh * hd + 2 * w;
                    if (g_ref16)
                    {
                        size_t dq = ((size_t)hh * S + s) * hd + 2 * w;
                        size_t dk = ((size_t)hh * ctx + offset + s) * hd + 2 * w;
                        oracle_rope16_pair(q[src], q[src + 1], offset + s, w, hd, c->theta, &rq[dq], &rq[dq + 1]);
                        oracle_rope16_pair(k[src], k[src + 1], offset + s, w, hd, c->theta, &kc[dk], &kc[dk + 1]);
                        vc[dk] = v[src];
                        vc[dk + 1] = v[src + 1];
                        continue;
                    }
                    float f = (float)(offset + s) / m->freqs[w];
                    float fc = cosf(f), fs = sinf(f);
                    float q0 = h2f(q[src]), q1 = h2f(q[src + 1]);
                    float k0 = h2f(k[src]), k1 = h2f(k[src + 1]);
                    size_t dq = ((size_t)hh * S + s) * hd + 2 * w;
                    rq[dq] = oracle_f32_to_f16(fc * q0 - fs * q1);
                    rq[dq + 1] = oracle_f32_to_f16(fs * q0 + fc * q1);
                    size_t dk = ((size_t)hh * ctx + offset + s) * hd + 2 * w;
                    kc[dk] = oracle_f32_to_f16(fc * k0 - fs * k1);
                    kc[dk + 1] = oracle_f32_to_f16(fs * k0 + fc * k1);
                    vc[dk] = v[src];
                    vc[dk + 1] = v[src + 1];
                }
        attn_job aj = {rq, kc, vc, att, S, offset, kv, D, hd, ctx, scale};
        par_for((size_t)H * S, attn_row, &aj, 2.0 * H * S * kv * hd);
        linear(att, (const uint16_t *)m->tensors[tid_blk(l, K_O)], o, S, D, D, 0);
        add_rows(h, o, (size_t)S * D);

        /* FFN sub-graph, src/models/vkllm_llama2_layers.c:13-96 */
        rmsnorm_rows(h, fn, xn, S, D, c->eps);
        linear(xn, (const uint16_t *)m->tensors[tid_blk(l, K_UP)], up, S, D, F, 0);
        linear(xn, (const uint16_t *)m->tensors[tid_blk(l, K_GATE)], gate, S, D, F, 1);
        for (size_t i = 0; i < (size_t)S * F; ++i)
            up[i] = oracle_f32_to_f16(h2f(up[i]) * h2f(gate[i]));
        uint16_t *down = o;
        linear(up, (const uint16_t *)m->tensors[tid_blk(l, K_DOWN)], down, S, F, D, 0);
        add_rows(h, down, (size_t)S * D);
    }

    /* output_norm -> logits for all S rows -> ARG_MAX (src/models/vkllm_models_llama2.c:561-587) */
    rmsnorm_rows(h, (const float *)m->tensors[tid_out_norm(c)], xn, S, D, c->eps);
    if (hidden_out)
        memcpy(hidden_out, xn, (size_t)S * D * 2);
    linear(xn, (const uint16_t *)m->tensors[tid_out(c)], logits, S, D, V, 0);
    oracle_tensor lt = {{1, 1, S, V}, {(uint32_t)(S * V), (uint32_t)(S * V), V, 1}, ORACLE_F16, logits};
    oracle_tensor ot = {{1, 1, S, 1}, {S, S, 1, 1}, ORACLE_U32, out_ids};
    oracle_arg_max(&lt, &ot);
    if (logits_out)
        memcpy(logits_out, logits, (size_t)S * V * 2);

    free(h);
    free(xn);
    free(q);
    free(k);
    free(v);
    free(rq);
    free(att);
    free(o);
    free(up);
    free(gate);
    free(logits);
    return 0;
}

int oracle_token_loop(oracle_model *m, const uint32_t *prompt, uint32_t P, uint32_t n_steps, uint32_t *out_ids,
                      uint16_t *last_logits)
{
    const uint32_t V = m->cfg.vocab;
    uint32_t offset = 0;
    uint32_t *ids = (uint32_t *)malloc(sizeof(uint32_t) * (P > 1 ? P : 1));
    uint16_t *lg = last_logits ? (uint16_t *)malloc((size_t)(P > 1 ? P : 1) * V * 2) : NULL;
    const uint32_t *in = prompt;
    uint32_t S = P, next = 0;
    for (uint32_t step = 0; step < n_steps; ++step)
    {
        if (oracle_model_step(m, in, S, offset, ids, lg, NULL) != 0)
        {
            free(ids);
            free(lg);
            return -1;
        }
        next = ids[S - 1];
        out_ids[step] = next;
        if (lg)
            memcpy(last_logits + (size_t)step * V, lg + (size_t)(S - 1) * V, (size_t)V * 2);
        offset += S;
        S = 1;
        in = &out_ids[step];
    }
    free(ids);
    free(lg);
    return 0;
}
