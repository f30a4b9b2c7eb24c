/* Extensions of this MI355X build that have no counterpart in the reference API. */
#ifndef VKLLM_HIP_H
#define VKLLM_HIP_H
#include <stdint.h>
#include "vkllm_errors.h"
#ifdef __cplusplus
extern "C" {
#endif

struct vkllm_context;
struct vkllm_graph;
struct vkllm_models_llama2;

/* How graphs built by vkllm_models_llama2_build_graph execute:
 * VKLLM_EXEC_FUSED (default): the whole token step as fused kernels; S == 1 steps replay a captured hipGraph.
 * VKLLM_EXEC_NODES: node by node through the VKLLM_OP_* kernels, every intermediate tensor materialised.
 * The environment variable VKLLM_EXEC=nodes|fused sets the initial mode of a context. */
#define VKLLM_EXEC_FUSED 0
#define VKLLM_EXEC_NODES 1
extern vkllm_err_t vkllm_hip_set_exec_mode(struct vkllm_context *context, int mode);
extern int vkllm_hip_get_exec_mode(struct vkllm_context *context);

/* 1: capture S == 1 fused steps into a hipGraph and replay it (default); 0: launch kernels directly */
extern vkllm_err_t vkllm_hip_set_graph_replay(struct vkllm_context *context, int enable);

/* per-launch hipEvent timing feeding vkllm_pipeline_query_exec_time and context->stats (also VKLLM_TIMING=1) */
extern vkllm_err_t vkllm_hip_set_timing(struct vkllm_context *context, int enable);

/* Number of kernel families (pipelines) of the library. */
extern int vkllm_hip_kernel_family_count(void);
/* Timing counters of kernel family `index` (0 <= index < vkllm_hip_kernel_family_count(), else VKLLM_ERR_ARGS):
 * its name, the number of timed launches and their summed duration in nanoseconds. Waits for pending launches. */
extern vkllm_err_t vkllm_hip_kernel_stats(struct vkllm_context *context, int index, const char **name,
                                          uint64_t *launches, uint64_t *total_ns);
/* Zeroes every kernel family's timing counters. */
extern vkllm_err_t vkllm_hip_reset_kernel_stats(struct vkllm_context *context);

/* Launches the decode-step kernel `family` `reps` times back to back, cycling over the layers' weights, between
 * one hipEvent pair on the context's stream, and returns the elapsed nanoseconds: the kernel's duration without
 * the per-launch dispatch latency that a per-launch event pair adds. Families: "fused_embed", "fused_qkv_rope",
 * "fused_attn_scores", "fused_attn_pv", "fused_attn_long" (both in one launch), "fused_attn_small", "fused_attn_o"
 * (one-kernel attention and Wo + residual in one launch), "fused_o_resid", "fused_gateup", "fused_down_resid",
 * "fused_logits", "fused_argmax" (the embedding and residual GEMVs write into a scratch row, so repeats leave the
 * model state unchanged), "decode_step": replays of the captured single-token graph the last step used, at
 * its position, and "decode_persist": the persistent single-token launch (VKLLM_PERSIST=1) recomputing the last
 * step, which must have run as that launch. Needs a preceding single-token step of `model`. */
extern vkllm_err_t vkllm_hip_model_time_kernel(struct vkllm_context *context, struct vkllm_models_llama2 *model,
                                               const char *family, uint32_t reps, uint64_t *total_ns);

/* Runs the VKLLM_OP_* operator of tensors[r % n] for r < reps back to back between one hipEvent pair on the
 * context's stream (each tensor is first run once outside the pair) and returns the elapsed nanoseconds: the ops'
 * kernel time without per-launch synchronisation. Several tensors with their own operands let a caller cycle through
 * more bytes than the GPU's caches hold. Per-launch timing (vkllm_hip_set_timing) is off inside the pair. */
extern vkllm_err_t vkllm_hip_time_ops(struct vkllm_context *context, struct vkllm_tensor *const *tensors, uint32_t n,
                                      uint32_t reps, uint64_t *total_ns);

/* Device figures for reading the roofline fractions (no counterpart in the reference; measurement entry points).
 * vkllm_hip_probe_stream_read: the HBM read rate, in GB/s (1e9 bytes per second), of a kernel that only streams
 * `window_bytes` with 16-byte non-temporal loads (each byte read once, nothing written), over windows of a 1 GiB
 * buffer that the call allocates and frees, so no window is found in the 256 MB memory-side cache; the median and
 * the best of `reps` timed passes (1..1024) after an untimed one. window_bytes is a multiple of 32 MiB, at most
 * 1 GiB.
 * vkllm_hip_probe_launch_gap: microseconds per launch of a chain of `launches` (1..4096) empty kernels of `blocks`
 * workgroups of 256 threads, each after the one before on the context's stream, captured into a hipGraph and
 * replayed as the decode step is: the cost of one kernel boundary. */
extern vkllm_err_t vkllm_hip_probe_stream_read(struct vkllm_context *context, uint64_t window_bytes, uint32_t reps,
                                               double *gbps_median, double *gbps_best);
extern vkllm_err_t vkllm_hip_probe_launch_gap(struct vkllm_context *context, uint32_t launches, uint32_t blocks,
                                              double *us_per_launch);

/* Model configuration for vkllm_models_llama2_init_random. */
struct vkllm_llama2_config
{
    uint32_t block_count;
    uint32_t embedding_length;
    uint32_t head_count;
    uint32_t feed_forward_length;
    uint32_t vocab_size;
    uint32_t context_length;
    float layer_norm_rms_epsilon;
    float rope_freq_base;
    float weight_std;
};

/* Builds a LLaMA-2 model whose weights are generated on the GPU from (config, seed) by the same definition the
 * oracle's random-init GGUF writer uses (Irwin-Hall normal of counter-based SplitMix64 words, times
 * weight_std, rounded to fp16; norm weights 1.0), so it equals loading that GGUF file, without the file.
 * Tokenizer metadata is left empty. */
extern vkllm_err_t vkllm_models_llama2_init_random(struct vkllm_context *context, struct vkllm_models_llama2 *model,
                                                   const struct vkllm_llama2_config *config, uint64_t seed);

/* Copies the fp16 logits [rows, vocab] of the model's last fused step into dst (rows <= that step's S). */
extern vkllm_err_t vkllm_hip_model_last_logits(struct vkllm_context *context, struct vkllm_models_llama2 *model,
                                               uint16_t *dst, uint32_t rows);

/* The reference driver's token loop (tests/vkllm_test_infer_gguf.c:181-272) in C: step 0 feeds `prompt`
 * (prompt_len ids) at position `offset0`, every later step the previous step's last arg-max id at the next
 * position. Each step runs vkllm_tensor_new(input_toks, mapped) -> vkllm_graph_new ->
 * vkllm_models_llama2_build_graph -> vkllm_graph_init -> vkllm_commands_upload -> vkllm_graph_run ->
 * vkllm_graph_post_run -> vkllm_tensor_invalid_cache -> read the last id -> vkllm_graph_free.
 * ids[i] receives step i's last arg-max id, step_ns[i] (optional) the step's wall time, and phase_ns[4] (optional)
 * the wall time summed over steps 1.. of: tensor_new + graph_new + build_graph; graph_init + upload;
 * graph_run + post_run; invalid_cache + read + graph_free. */
extern vkllm_err_t vkllm_hip_token_loop(struct vkllm_context *context, struct vkllm_models_llama2 *model,
                                        const uint32_t *prompt, uint32_t prompt_len, uint32_t offset0,
                                        uint32_t n_steps, uint32_t *ids, uint64_t *step_ns, uint64_t *phase_ns);

/* The prompt-step GEMM on caller-owned device memory, on the context's stream; returns when C is written.
 * C[M, N] (row stride ldc >= N) = A[M, K] . B[N, K]^T with fp16 operands and fp32 accumulation (K % 8 == 0; A, B
 * and work 16-byte aligned), then the epilogue `epi`: 0 C = fp16(acc); 1 columns >= split fp16(silu(acc)), the
 * others fp16(acc); 2 C = fp16(C + fp16(acc)) (C holds the residual on entry); 3 (B = [Wu; Wg] with split = F rows
 * each, N = 2F, N % 64 == 0, K % 64 == 0, ldc >= F, ldc % 8 == 0, C 16-byte aligned) C[m][f] =
 * fp16(fp16(A[m] . Wu[f]) * fp16(silu(A[m] . Wg[f]))), the FFN's SwiGLU, for f < F. `work` (work_elems floats,
 * device memory, may be NULL with work_elems 0) holds split-K partial tiles; with too little of it K is not split.
 * Arguments outside these rules return VKLLM_ERR_ARGS. This is the kernel behind the
 * fused step's matmul nodes (src/core/vkllm_op_matmul.c), exposed so that its tile and split choices can be checked
 * and timed at any shape. */
extern vkllm_err_t vkllm_hip_gemm(struct vkllm_context *context, int epi, const uint16_t *A, const uint16_t *B,
                                  uint16_t *C, uint32_t M, uint32_t N, uint32_t K, uint32_t ldc, uint32_t split,
                                  float *work, uint64_t work_elems);

/* The short-prompt product of the fused step (prompts of at most 128 tokens), with vkllm_hip_gemm's arguments and
 * epilogues 0 (C = fp16(acc), ldc >= N), 2 (C = fp16(C + fp16(acc)), ldc == N, N % 32 == 0) and 3 (the SwiGLU of
 * B = [Wu; Wg], N = 2F, F % 16 == 0, ldc >= F); M <= 128, K % 16 == 0, A and B 16-byte aligned, C 8-byte aligned,
 * ldc % 4 == 0. It copies B into the fragment-tiled layout the fused step keeps for its weights and A into
 * fragment order (allocating both), then streams the weights through the matrix cores; `splits` (at most 8; 0 for
 * the fused step's choice) sets the K ranges of epilogue 2. Returns when C is written. There is no counterpart in
 * the reference: this exposes the kernel behind the fused step's short-prompt matmul nodes for checks and timing. */
extern vkllm_err_t vkllm_hip_gemm_streamed(struct vkllm_context *context, int epi, const uint16_t *A,
                                           const uint16_t *B, uint16_t *C, uint32_t M, uint32_t N, uint32_t K,
                                           uint32_t ldc, uint32_t splits);

/* vkllm_hip_gemm for callers that cannot allocate device memory (code under stream capture, serving loops that
 * forbid hipMalloc). It has no counterpart in the reference. The split-K partial tiles go to a fixed scratch array
 * of the library (8M floats, 32 MiB, held by every GPU the library runs on until the process ends) instead of a
 * caller buffer: `work_elems` (at most 8M, else VKLLM_ERR_ARGS) is how much of it the product may use, with the
 * meaning of vkllm_hip_gemm's work_elems, so the same arguments give the same tile and split choices and identical
 * results. The call enqueues on the context's stream and returns without waiting (vkllm_hip_synchronize waits); it
 * calls no allocating routine. Calls queued on one stream run in order; calls from two contexts on one GPU at once
 * race on the shared scratch. */
extern vkllm_err_t vkllm_hip_gemm_noalloc(struct vkllm_context *context, int epi, const uint16_t *A,
                                          const uint16_t *B, uint16_t *C, uint32_t M, uint32_t N, uint32_t K,
                                          uint32_t ldc, uint32_t split, uint64_t work_elems);

/* The HIP stream (a hipStream_t) every call on the context enqueues on: the stream a caller captures into a
 * hipGraph around vkllm_hip_gemm_noalloc, or orders its own work against. */
extern vkllm_err_t vkllm_hip_context_stream(struct vkllm_context *context, void **stream);

/* Synchronise the context's stream. */
extern vkllm_err_t vkllm_hip_synchronize(struct vkllm_context *context);

/* Name of the device (hipDeviceProp_t::gcnArchName) for logs. */
extern const char *vkllm_hip_device_arch(struct vkllm_context *context);

/* Layout facts for FFI bindings: sizeof and field offsets of the public structs. Returns the number of
 * entries written (at most n); `names` receives static strings. */
extern int vkllm_hip_abi_layout(const char **names, uint64_t *values, int n);

#ifdef __cplusplus
}
#endif
#endif
