/*
 * CPU oracle for the vkllm.c LLaMA-2 token loop.
 *
 * TEST INFRASTRUCTURE ONLY. Nothing in the shipped library links, loads or calls this code; only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg use it, and only to check the library's results.
 *
 * It restates, in plain C, the semantics of the reference's operators and of its LLaMA-2 graph. Each function
 * cites the reference file:line it follows (paths relative to the vkllm.c tree).
 *
 * Numerics mode: fp16 storage, fp32 arithmetic -- the variant the reference selects when the device has 16-bit
 * storage but no fp16 arithmetic (src/core/vkllm_op_matmul.c:103-113, src/shaders/BUILD:82,102,121,141). A second
 * mode (REF16, oracle_set_numerics below) restates the fp16-arithmetic variants to measure how far they drift.
 * Every graph node's output is rounded to its storage dtype (fp16 round-to-nearest-even), exactly where the
 * reference's graph materialises a tensor. Reductions (dot products, sums of squares, softmax sums) are
 * accumulated in double and rounded once to fp32: the reference's fp32 summation order is decided by the
 * Vulkan driver (subgroupAdd, dot()) and is not pinned by anything in its sources, so the oracle uses the
 * order-free value that every fp32 order approximates.
 *
 * Tensors are described by oracle_tensor: 4-D [N, C, H, W] shapes, strides in ELEMENTS (the reference keeps
 * byte strides in struct vkllm_tensor, src/core/vkllm_tensor.c:13-31, and divides them by the element size
 * before dispatch, e.g. src/core/vkllm_op_matmul.c:168-171).
 */
#ifndef VKLLM_ORACLE_H
#define VKLLM_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* dtype codes are the reference's (src/core/vkllm_dtypes.inc:5-8) */
enum
{
    ORACLE_F32 = 1,
    ORACLE_F16 = 2,
    ORACLE_I8 = 3,
    ORACLE_U32 = 4
};

typedef struct
{
    uint32_t shapes[4];
    uint32_t strides[4]; /* elements */
    int32_t dtype;
    void *data;
} oracle_tensor;

/* ---- fp16 <-> fp32 (IEEE binary16, round-to-nearest-even, subnormals kept) ---- */
uint16_t oracle_f32_to_f16(float f);
float oracle_f16_to_f32(uint16_t h);

/* ---- counter-based random numbers used for every synthetic input ----
 * splitmix64 finaliser of (stream + (n+1) * 0x9E3779B97F4A7C15): the n-th output of a SplitMix64 generator
 * whose state starts at `stream`. */
uint64_t oracle_splitmix64(uint64_t stream, uint64_t n);
/* approximately N(0,1): Irwin-Hall sum of 12 uniforms taken as 16-bit fields of three splitmix64 outputs,
 * computed exactly: z = (sum_k b_k + 6 - 6*65536) / 65536 with b_k in [0, 65535]. */
float oracle_normal(uint64_t stream, uint64_t i);
/* weight i of random tensor number `tensor_id` under `seed`: fp16(oracle_normal(...) * std) */
uint16_t oracle_weight_f16(uint64_t seed, uint32_t tensor_id, uint64_t i, float std);
uint64_t oracle_tensor_stream(uint64_t seed, uint32_t tensor_id);
/* prompt token i under `seed`: splitmix64(seed, i) % vocab */
uint32_t oracle_prompt_token(uint64_t seed, uint32_t i, uint32_t vocab);

/* ---- operators (return 0 on success, -1 on a shape/dtype error) ---- */

/* src/core/vkllm_op_matmul.c:14-24 */
int oracle_is_transposed_b(const oracle_tensor *a, const oracle_tensor *b, const oracle_tensor *out);

/* VKLLM_OP_MATMUL: out = act(scale * A . B) with B [N,K] when oracle_is_transposed_b(), else [K,N].
 * Batch dims of size 1 broadcast. act 1 = SiLU v/(1+exp(-v)).
 * src/core/vkllm_op_matmul.c:32-63,317-329, src/shaders/vkllm_mat_mul_vec.comp:94-150,
 * src/shaders/vkllm_matmul_t1.comp:90-251, src/shaders/vkllm_matmul_t0.comp:92-245 */
int oracle_matmul(const oracle_tensor *a, const oracle_tensor *b, oracle_tensor *out, float scale, int32_t act);

/* VKLLM_OP_EMBEDDING: src/core/vkllm_op_embedding.c:40-55, src/shaders/vkllm_embedding.comp:41-70 */
int oracle_embedding(const oracle_tensor *idx, const oracle_tensor *table, oracle_tensor *out, uint32_t unk_tok);

/* VKLLM_OP_RMSNORM: y = (x*w) * 1/sqrt(sum(x^2)/W + eps); src/shaders/vkllm_rmsnorm.comp:31-82 */
int oracle_rmsnorm(const oracle_tensor *x, const oracle_tensor *w, oracle_tensor *out, float eps);

/* VKLLM_OP_ROPE: src/shaders/vkllm_rope.comp:39-79; angle (offset+h) / freqs[w] with freqs from oracle_rope_freqs */
int oracle_rope(const oracle_tensor *in, oracle_tensor *out, uint32_t offset, float base, int neox_style);
/* denominators base^(2w/D) for w in [0, D/2), computed with the C library's powf */
void oracle_rope_freqs(float base, uint32_t D, float *freqs);

/* VKLLM_OP_SOFTMAX: src/shaders/vkllm_softmax.comp:42-96 (input addressed with the OUTPUT strides,
 * src/core/vkllm_op_softmax.c:71-81) */
int oracle_softmax(const oracle_tensor *in, oracle_tensor *out, int32_t seq_mask, uint32_t offsets);

/* VKLLM_OP_UPDATE_ROWS: cache[b,c,h+off,w] = src[b,c,h,w]; src/shaders/vkllm_update_rows.comp:21-46 */
int oracle_update_rows(const oracle_tensor *src, oracle_tensor *cache, uint32_t offset_rows);

/* VKLLM_OP_COPY: strided gather; src/shaders/vkllm_copy.comp:35-50 */
int oracle_copy(const oracle_tensor *in, oracle_tensor *out);

/* VKLLM_OP_BIN: op 0 add, 1 sub, 2 mul, 3 div; all three tensors addressed with the OUTPUT strides
 * (src/shaders/vkllm_bin_op.comp:41-73, src/core/vkllm_op_bin.c:60-90) */
int oracle_bin(const oracle_tensor *a, const oracle_tensor *b, oracle_tensor *out, int32_t op);

/* VKLLM_OP_ARG_MAX: the 32-lane scan + strict-> tree of src/shaders/vkllm_arg_max.comp:40-97 */
int oracle_arg_max(const oracle_tensor *in, oracle_tensor *out);

/* VKLLM_OP_FFN_UP_AND_GATE: out = (x.Wu^T) * silu(x.Wg^T); src/shaders/vkllm_ffn_up_and_gate.comp:44-149 */
int oracle_ffn_up_and_gate(const oracle_tensor *x, const oracle_tensor *wu, const oracle_tensor *wg,
                           oracle_tensor *out);

/* ---- REF16: the reference's fp16-arithmetic shader variants ----
 * With fp16 arithmetic on the device the reference selects the f16f16 variants (src/core/vkllm_op_matmul.c:92-101,
 * src/core/vkllm_op_rope.c:22, src/core/vkllm_op_softmax.c:24; macros at src/shaders/BUILD:81,101,120,140) instead
 * of the fp32-arithmetic ones the library follows. The residual adds and the up * gate product (bin_op f16f16f16,
 * src/shaders/BUILD:24) round one fp16 operation and RMSNorm has no fp16-arithmetic variant (BUILD:55-68), so those
 * are as in the fp32 mode. REF16
 * restates them: every arithmetic operation on fp16 values rounds its exact result once to fp16 (round to nearest
 * even; fp16 exp, cos, sin and pow are the correctly rounded values), and the driver-defined parts take one fixed
 * choice: subgroupAdd adds the lanes in order, dot(f16vec2) is fp16(fp16(a0 b0) + fp16(a1 b1)), and dot(vec4) in
 * fp32 adds the four products in order. Nothing in the reference pins those choices, so REF16 measures how far an
 * fp16-arithmetic device's tokens and logits can be from the fp32-arithmetic ones; it is not a bit-exact restatement.
 * oracle_set_numerics(1, g) switches the model step to it with subgroups of g lanes (lavapipe's width on the host
 * CPU; 32 in the shader's comments); oracle_set_numerics(0, 0) restores the fp32 mode. Not thread-safe: set it
 * between steps. */
void oracle_set_numerics(int ref16, uint32_t subgroup);
/* Summation order of the fp32 mode's model step (projections, RMSNorm sums of squares, attention scores, softmax
 * sums, P.V). 0 (the default): sums in double, rounded once to fp32, the stand-in for an exact sum that every fp32
 * order approximates. 1: sums in fp32, one term at a time in index order, the least accurate of the usual orders.
 * Every rounding to fp16 stays where the reference's graph materialises a tensor; only the sums change. The
 * reference's own order is its driver's (subgroup trees, tile loops) and nothing pins it, so the distance between
 * these two orders' outputs is the scale on which a third valid order is judged where one-ulp fp16 differences
 * accumulate through many layers. Not thread-safe: set it between steps. */
void oracle_set_accumulation(int fp32_sequential);
/* fp16 round-to-nearest-even of a double (no double rounding through fp32) */
uint16_t oracle_f64_to_f16(double v);
/* src/shaders/vkllm_mat_mul_vec.comp:118-146 f16f16: one output of x[K] . w[K] (K % 4 == 0), times scale, SiLU
 * when act, in fp16 with subgroups of `subgroup` lanes */
uint16_t oracle_gemv16(const uint16_t *x, const uint16_t *w, uint32_t K, float scale, int act, uint32_t subgroup);
/* src/shaders/vkllm_matmul_t1.comp:202-221 f16f16f16: sum over k pairs of fp16 dot(f16vec2), accumulated in fp32
 * (an odd K pads the last pair with 0); returns the fp32 sum */
float oracle_gemm16_dot(const uint16_t *a, const uint16_t *b, uint32_t K);
/* src/shaders/vkllm_softmax.comp:53-95 f16f16 on one row of W fp16 values: entries i > limit masked (limit >= W:
 * none) */
void oracle_softmax16_row(const uint16_t *x, uint16_t *out, uint32_t W, uint32_t limit, uint32_t subgroup);
/* src/shaders/vkllm_rope.comp:68-78 f16f16: pair (v0, v1) at dims (2w, 2w + 1) of a head of size hd at position
 * pos rotated with fp16 angle arithmetic */
void oracle_rope16_pair(uint16_t v0, uint16_t v1, uint32_t pos, uint32_t w, uint32_t hd, float base, uint16_t *o0,
                        uint16_t *o1);

/* ---- LLaMA-2 model ---- */
typedef struct
{
    uint32_t n_layer;
    uint32_t dim;
    uint32_t n_head;
    uint32_t n_head_kv;
    uint32_t ffn;
    uint32_t vocab;
    uint32_t ctx;
    float eps;
    float theta;
    uint32_t bos_id;
    uint32_t eos_id;
    uint32_t pad_id;
    float weight_std;
} oracle_llama_cfg;

/* Random-init GGUF v3 file: every matrix fp16 oracle_weight_f16(seed, id, i, std), norm weights F32 1.0.
 * Tensor ids follow the write order: token_embd 0; block l: attn_norm, attn_q, attn_k, attn_v, attn_output,
 * ffn_norm, ffn_gate, ffn_up, ffn_down = 1+9l .. 9+9l; output_norm 1+9L; output 2+9L.
 * Keys are the ones src/models/vkllm_models_llama2.c:78-183 reads, plus a small synthetic tokenizer. */
int oracle_gguf_write_random(const char *path, const oracle_llama_cfg *cfg, uint64_t seed);

typedef struct oracle_model oracle_model;
/* GGUF reader independent of the library's: src/models/vkllm_models_llama2.c:189-253,255-412 */
oracle_model *oracle_model_load(const char *path);
/* same model built directly from (cfg, seed) without a file */
oracle_model *oracle_model_random(const oracle_llama_cfg *cfg, uint64_t seed);
void oracle_model_free(oracle_model *m);
int oracle_model_cfg(const oracle_model *m, oracle_llama_cfg *cfg);
/* weights of tensor `tensor_id` (fp16 matrices) or NULL */
const uint16_t *oracle_model_weight(const oracle_model *m, uint32_t tensor_id, size_t *count);

/* One call of vkllm_models_llama2_build_graph + graph run for S tokens at `offset`
 * (src/models/vkllm_models_llama2.c:488-602, src/models/vkllm_llama2_layers.c:13-354).
 * Writes the S argmax ids; optional fp16 logits [S, vocab] and fp16 final hidden state [S, dim]. */
int oracle_model_step(oracle_model *m, const uint32_t *toks, uint32_t S, uint32_t offset, uint32_t *out_ids,
                      uint16_t *logits, uint16_t *hidden);

/* The token loop of tests/vkllm_test_infer_gguf.c:173-272: prefill `prompt`, then keep feeding the argmax of
 * the last row. Writes n_steps ids (the first is the prefill's). Optional logits of the last row per step. */
int oracle_token_loop(oracle_model *m, const uint32_t *prompt, uint32_t P, uint32_t n_steps, uint32_t *out_ids,
                      uint16_t *last_logits);

#ifdef __cplusplus
}
#endif
#endif
