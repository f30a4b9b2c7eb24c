// Fused execution of a LLaMA-2 token step built by vkllm_models_llama2_build_graph.
//
// The graph keeps the reference's node structure (src/models/vkllm_models_llama2.c:488-602); its plan records
// (model, input ids, offset, S). Running the plan:
//   S == 1  the decode step: embed, 6 fused kernels per layer, logits, arg max. Kernels read the position from a
//           device-resident Step, so the whole sequence is captured once per model as a hipGraph and replayed for
//           every token. The token id and position reach the device through a coherent pinned host block that
//           the first kernel reads; the arg max writes the chosen id back into it, so no copy is queued.
//   S >  1  prefill: embed, per layer RMSNorm -> QKV GEMM (MFMA) -> RoPE + KV append -> attention -> Wo GEMM with
//           the residual add -> RMSNorm -> [up;gate] GEMM with SiLU on the gate half -> up*gate -> Wd GEMM with
//           the residual add; then RMSNorm -> logits GEMM for all S rows -> arg max per row.
// Either way the S arg-max ids land in the mapped output tensor, as the reference's ARG_MAX node leaves them.
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <ctime>
#include <string>
#include <unordered_map>
#include <vector>

#include "model_priv.h"

struct FusedPlan
{
    vkllm_models_llama2 *model;
    vkllm_tensor *input_toks;
    uint32_t offset;
    uint32_t S;
    bool ran = false; // fused_plan_run enqueued (and completed) the step
};

// Short-cache decode steps are captured per bucket of kSmallBucket cache positions: a bucket's launches bound their
// LDS and the keys and V rows they request before the position is known by the bucket's end.
constexpr uint32_t kSmallBucket = 64, kSmallBuckets = 24;

struct FusedState
{
    uint32_t cap_S = 0; // rows the activation buffers hold
    uint16_t *h = nullptr, *xn = nullptr, *qkv = nullptr, *q = nullptr, *attn = nullptr, *act = nullptr,
             *ug = nullptr, *logits = nullptr;
    uint32_t *ids = nullptr, *toks = nullptr;
    float *rope_cs = nullptr;    // a prompt step's RoPE angles [S][hd / 2][2], shared by its layers
    vk::Step *step = nullptr;    // device
    vk::Step *step_h = nullptr;  // pinned staging for step + first token
    uint32_t *io_h = nullptr;    // pinned: a prefill's ids, uploaded and read back
    // single-token steps alternate between two slots, so that the next step can be enqueued while the host still
    // reads this one (launch-ahead, below). Each slot has a pinned coherent DecodeIo (position, token, arg-max id),
    // a device copy of its arg-max id, a logits row and its own captured graphs; `dio` and `slot` name the slot
    // being enqueued
    vk::DecodeIo *dio_slots = nullptr; // [2]
    vk::DecodeIo *dio = nullptr;
    uint32_t *slot_ids = nullptr;      // [2], device
    uint16_t *slot_logits = nullptr;   // [2][V], device
    int slot = 0;
    hipEvent_t slot_done[2] = {};      // recorded after each slot's last launch
    // Launch-ahead (VKLLM_LAUNCH_AHEAD=0: off). After enqueueing a single-token step at position p, the step at p + 1
    // is enqueued behind it with the first step's device-side arg max as its token, before the host has read that id.
    // The reference driver's loop feeds exactly that id back at p + 1 (tests/vkllm_test_infer_gguf.c:255-269), so its
    // next graph_run finds the step already queued or done and only waits. Any other next call (another token or
    // position, a prompt step, timing) discards the step launched ahead, whose only lasting effect is the cache rows
    // of position p + 1: a step at that position rewrites them before reading them, and no step reads a row past its
    // own position.
    bool ahead_enabled = true;
    bool ahead_live = false;
    int ahead_slot = 0;
    uint32_t ahead_offset = 0, ahead_token = 0; // the step launched ahead: its position, and its token once known
    // the last completed single-token step (what vkllm_hip_model_last_logits and the timing replays refer to)
    int done_slot = 0;
    uint32_t done_offset = 0, done_token = 0;
    const uint16_t *last_logits = nullptr; // logits of the last completed step (a slot's row, or the prompt's rows)
    float *freqs = nullptr;      // device copy of the RoPE denominators
    // decode attention scratch: scores [H, ctx], chunk statistics [H, cmax, 2], chunk partial sums [H, cmax, hd]
    float *att_scores = nullptr, *att_stats = nullptr, *att_part = nullptr;
    uint32_t *att_count = nullptr; // per-head chunk arrivals of the merge, zero between launches
    uint32_t *attn_sync = nullptr; // counters and flags of the attention + projection launch, zero between launches
    uint32_t *att_long_sync = nullptr; // per-head counters of the one-kernel long-cache attention, zero between launches
    float *gemm_work = nullptr;    // split-K partial tiles of short-prompt prefill GEMMs
    // a single-token step's arg max in the vocabulary product's epilogue (VKLLM_ARGMAX_EPI=0: a separate kernel):
    // per-workgroup candidates and the arrival counter (zero between launches); cleared when the product's shape
    // does not take that epilogue
    bool argmax_epi = true;
    float *am_val = nullptr;
    uint32_t *am_idx = nullptr, *am_count = nullptr;
    // prompt steps of at most 128 tokens (VKLLM_PREFILL_TILED=0: off): fragment-tiled copies of the QKV, output,
    // gate/up and vocabulary matrices (one slab), streamed by launch_stream_gemm, and the fragment-ordered
    // activations it reads ([128, D] each: the normalised rows and the attention output)
    bool stream_ok = false, stream_tried = false;
    void *tile_slab = nullptr;
    struct Tiles
    {
        uint16_t *wqkv, *wo, *wug;
    };
    std::vector<Tiles> tiles;
    uint16_t *out_t = nullptr, *xn_t = nullptr, *attn_t = nullptr;
    uint32_t att_cmax = 0, att_chunk = 0;
    uint32_t attn_max_groups = 8; // dim slices per head of the short-cache attention, at most (VKLLM_ATTN_GROUPS)
    // decode attention in one kernel up to this many positions, in two kernels beyond (VKLLM_ATTN_SMALL_MAX)
    uint32_t attn_small_max = 0;
    // one-kernel attention and the output projection in one launch (VKLLM_ATTN_O=1; the default is two launches,
    // which measure faster at the 7B widths); cleared when the device cannot hold both parts' workgroups at once
    bool attn_o = false;
    // short caches of at most kAttnTailMaxKv positions: each head's attention at the end of the QKV product, by the
    // workgroup that completes the head's rows (VKLLM_QKV_ATTN=1; the default is the separate attention kernel,
    // which measures faster at the 7B widths: every head completes in the product's last round, so the attention's
    // latency follows the product in one 256-thread workgroup per head). head_count: the product's per-head unit
    // counts, zero between launches.
    bool qkv_attn = false, qkv_attn_now = false;
    uint32_t *head_count = nullptr;
    // single-token steps with short caches as one persistent launch after the embedding (VKLLM_PERSIST=1; the
    // default is the separate kernels, which measure faster at the 7B shape); cleared when a wait of that launch
    // gives up or the device cannot hold its grid. Its activations: the residual stream [2L + 1] rows, q, attention
    // output [L] rows, FFN activations [L] rows (each row written once per step), the layers' weight pointers, and
    // the barrier words (zero between launches).
    bool persist = false;
    vk::PersistLayer *persist_layers = nullptr;
    uint16_t *p_hs = nullptr, *p_qs = nullptr, *p_attns = nullptr, *p_acts = nullptr;
    uint32_t p_hstride = 0, p_fstride = 0;
    uint32_t *persist_sync = nullptr;
    bool p_variant[kSmallBuckets + 1] = {}; // per attention variant: its steps are enqueued as the persistent launch
    // long caches in one attention kernel (VKLLM_ATTN_LONG=0: two); cleared when the device cannot hold every chunk
    // block at once
    bool attn_long = true;
    // prompt steps: RoPE and the K/V append in the QKV product's epilogue where the shape allows it
    // (VKLLM_ROPE_EPI=0: the stored product and a separate kernel)
    bool rope_epi = true;
    // prompt steps: the RMSNorm after each residual product in its split-K reduce (VKLLM_NORM_EPI=0: a separate pass)
    bool norm_epi = true;
    // polls of the bounded waits before they give up (VKLLM_SPIN_LIMIT; 0 forces the give-up path)
    uint32_t long_spin_limit = vk::kAttnLongSpinLimit, attn_o_spin_limit = vk::kAttnOSpinLimit;
    // captured single-token steps, one per attention variant: [b] (b < kSmallBuckets) the one-kernel attention for
    // caches of at most (b + 1) * kSmallBucket positions (the launch's bound for its LDS and speculative loads),
    // [kSmallBuckets] the long-cache attention
    hipGraph_t graph[2][kSmallBuckets + 1] = {};
    hipGraphExec_t exec[2][kSmallBuckets + 1] = {};
    // the positions bound of the short-cache launches being enqueued (the current variant's)
    uint32_t small_kv_max = 0;
    int last_exec = -1, last_exec_slot = 0;
    // timing mode: one record per graph node a fused launch computes (per layer, then the step's own nodes), named
    // as the node; after a timed step the graph's nodes point at the records that received launches
    std::vector<vkllm_pipeline> node_pipes;
    std::vector<std::string> node_names;
    std::unordered_map<std::string, int> node_index;
    // VKLLM_TRACE_HOST=1: host time of single-token steps spent enqueueing and waiting, printed at release
    bool trace = false;
    uint64_t trace_steps = 0, trace_enqueue_ns = 0, trace_wait_ns = 0;
};

// Graph nodes (src/models/vkllm_llama2_layers.c:98-354, src/models/vkllm_models_llama2.c:488-602) that the fused
// launches are charged to in timing mode: the node a launch computes, or the first of the nodes it computes.
enum NodeSlot
{
    NS_ATTN_NORM = 0, // block.l.attn.norm: the prompt step's RMSNorm pass
    NS_Q,             // block.l.attn.Q: the QKV product (with RMSNorm, RoPE and the K/V append where fused)
    NS_RQ,            // block.l.attn.RQ: the separate RoPE + K/V append
    NS_RK,            // block.l.attn.RK: the prompt step's RoPE angle table (layer 0)
    NS_SCORES,        // block.l.attn.scores: attention (scores, softmax, P.V) in one launch, or its scores part
    NS_ATTN,          // block.l.attn: the P.V part of a two-launch attention
    NS_WO,            // block.l.attn.final_output: Wo + residual
    NS_FFN_NORM,      // block.l.ffn.norm
    NS_UP,            // block.l.ffn.up: the up/gate product with SwiGLU
    NS_MUL,           // block.l.ffn.mul: the separate SwiGLU
    NS_DOWN,          // block.l.ffn.down: Wd + residual
    NS_PER_LAYER,
    // the step's own nodes, after the layers
    NS_EMBEDDED = 0,
    NS_OUTPUT_NORM,
    NS_LOGITS,
    NS_OUTPUT,
    NS_GLOBAL
};

static void make_node_records(FusedState *fs, uint32_t L)
{
    static const char *per_layer[NS_PER_LAYER] = {"attn.norm", "attn.Q",  "attn.RQ",  "attn.RK",  "attn.scores", "attn",
                                                  "attn.final_output", "ffn.norm", "ffn.up", "ffn.mul", "ffn.down"};
    static const char *global[NS_GLOBAL] = {"embedded", "output_norm", "logits", "output"};
    const size_t n = (size_t)L * NS_PER_LAYER + NS_GLOBAL;
    fs->node_names.reserve(n);
    for (uint32_t l = 0; l < L; ++l)
        for (int k = 0; k < NS_PER_LAYER; ++k)
            fs->node_names.push_back("block." + std::to_string(l) + "." + per_layer[k]);
    for (int k = 0; k < NS_GLOBAL; ++k)
        fs->node_names.push_back(global[k]);
    fs->node_pipes.assign(n, vkllm_pipeline{});
    for (size_t i = 0; i < n; ++i)
    {
        fs->node_pipes[i].name = fs->node_names[i].c_str();
        fs->node_pipes[i].kernel_id = -1;
        fs->node_index.emplace(fs->node_names[i], (int)i);
    }
}

// the next timed launch is charged to node `slot` of layer l (or, with l == UINT32_MAX, the step's node `slot`)
static void charge(vkllm_context *ctx, FusedState *fs, int slot, uint32_t l = UINT32_MAX)
{
    if (!ctx->device->timing || fs->node_pipes.empty())
        return;
    const size_t L = (fs->node_pipes.size() - NS_GLOBAL) / NS_PER_LAYER;
    ctx->device->timing_node = &fs->node_pipes[l == UINT32_MAX ? L * NS_PER_LAYER + slot : (size_t)l * NS_PER_LAYER + slot];
}

// split-K workspace of the prefill GEMMs: 64 MB of fp32 partial tiles (4 splits of a 128-row QKV product at
// dim 5120 need 31 MB)
static constexpr size_t kGemmWorkElems = (size_t)16 << 20;
// workgroups of the vocabulary product with the arg-max epilogue, at most (one candidate each)
static constexpr uint32_t kArgmaxCandidates = 4096;

static uint64_t host_ns()
{
    timespec ts;
    clock_gettime(CLOCK_MONOTONIC, &ts);
    return (uint64_t)ts.tv_sec * 1000000000ull + (uint64_t)ts.tv_nsec;
}

void *fused_plan_new(vkllm_models_llama2 *model, vkllm_tensor *input_toks, uint32_t offset)
{
    auto *p = new FusedPlan();
    p->model = model;
    p->input_toks = input_toks;
    p->offset = offset;
    p->S = input_toks->shapes[3];
    return p;
}

bool fused_plan_ran(const void *plan)
{
    return ((const FusedPlan *)plan)->ran;
}

void fused_plan_free(void *plan)
{
    delete (FusedPlan *)plan;
}

static void free_stream_tiles(FusedState *fs)
{
    void *bufs[] = {fs->tile_slab, fs->xn_t, fs->attn_t};
    for (void *b : bufs)
        if (b)
            (void)hipFree(b);
    fs->tile_slab = nullptr;
    fs->xn_t = fs->attn_t = nullptr;
    fs->out_t = nullptr;
    fs->tiles.clear();
    fs->stream_ok = false;
}

static void free_buffers(FusedState *fs)
{
    void *bufs[] = {fs->h, fs->xn, fs->qkv, fs->q, fs->attn, fs->act, fs->ug, fs->logits, fs->ids, fs->toks,
                    fs->rope_cs};
    for (void *b : bufs)
        if (b)
            (void)hipFree(b);
    fs->h = fs->xn = fs->qkv = fs->q = fs->attn = fs->act = fs->ug = fs->logits = nullptr;
    fs->rope_cs = nullptr;
    fs->ids = fs->toks = nullptr;
    fs->cap_S = 0;
}

static void drop_graphs(FusedState *fs)
{
    for (int k = 0; k < 2; ++k)
        for (uint32_t i = 0; i <= kSmallBuckets; ++i)
        {
            if (fs->exec[k][i])
                (void)hipGraphExecDestroy(fs->exec[k][i]);
            if (fs->graph[k][i])
                (void)hipGraphDestroy(fs->graph[k][i]);
            fs->exec[k][i] = nullptr;
            fs->graph[k][i] = nullptr;
        }
    fs->last_exec = -1;
}

void fused_model_release(vkllm_context *ctx, vkllm_models_llama2 *model)
{
    ModelPriv *mp = model_priv(model);
    if (!mp || !mp->fs)
        return;
    FusedState *fs = mp->fs;
    (void)hipStreamSynchronize(ctx->device->stream);
    if (fs->trace && fs->trace_steps)
        fprintf(stderr, "vkllm: %llu single-token steps: enqueue %.1f us, wait %.1f us per step\n",
                (unsigned long long)fs->trace_steps, fs->trace_enqueue_ns / 1e3 / fs->trace_steps,
                fs->trace_wait_ns / 1e3 / fs->trace_steps);
    drop_graphs(fs);
    free_buffers(fs);
    if (fs->step)
        (void)hipFree(fs->step);
    if (fs->freqs)
        (void)hipFree(fs->freqs);
    free_stream_tiles(fs);
    void *att[] = {fs->att_scores, fs->att_stats, fs->att_part, fs->att_count, fs->attn_sync, fs->att_long_sync,
                   fs->gemm_work,  fs->am_val,    fs->am_idx,   fs->am_count,  fs->head_count,
                   fs->persist_layers, fs->p_hs,     fs->p_qs,     fs->p_attns,   fs->p_acts,
                   fs->persist_sync};
    for (void *b : att)
        if (b)
            (void)hipFree(b);
    if (fs->step_h)
        (void)hipHostFree(fs->step_h);
    if (fs->io_h)
        (void)hipHostFree(fs->io_h);
    if (fs->dio_slots)
        (void)hipHostFree(fs->dio_slots);
    if (fs->slot_ids)
        (void)hipFree(fs->slot_ids);
    if (fs->slot_logits)
        (void)hipFree(fs->slot_logits);
    for (hipEvent_t e : fs->slot_done)
        if (e)
            (void)hipEventDestroy(e);
    delete fs;
    mp->fs = nullptr;
}

// The fragment-tiled weight copies of the short-prompt products, made from the slab at the first prompt step of at
// most 128 tokens (decode-only use never pays for them). Shapes the streamed products and their producers cannot
// take, too little free memory, or a failed allocation leave stream_ok false: those steps then run on the row-major
// slab.
static vkllm_err_t build_stream_tiles(vkllm_context *ctx, ModelPriv *mp)
{
    FusedState *fs = mp->fs;
    fs->stream_tried = true;
    const char *e = getenv("VKLLM_PREFILL_TILED");
    if (e && *e == '0')
        return VKLLM_ERR_OK;
    const uint32_t D = mp->D, F = mp->F, V = mp->V, hd = mp->hd;
    // the QKV product's RoPE epilogue, the MFMA attention's fragment-ordered output, the interleaved gate/up rows
    if (D % 64 != 0 || F % 16 != 0 || hd < 32 || (hd & (hd - 1)) != 0 || !vk::attn_prefill_mfma_ok(hd))
        return VKLLM_ERR_OK;
    const size_t per_layer = vk::stream_tiled_elems(3 * D, D, 0) + vk::stream_tiled_elems(D, D, 0) +
                             vk::stream_tiled_elems(2 * F, D, F);
    const size_t total = per_layer * mp->L + vk::stream_tiled_elems(V, D, 0);
    size_t free_b = 0, total_b = 0;
    HIP_TRY(hipMemGetInfo(&free_b, &total_b));
    if (total * 2 + (size_t)2 * 128 * D * 2 > free_b / 2)
    {
        log_error("short-prompt tiled weights need %.1f GB; %.1f GB free: prompt steps run on the row-major weights",
                  total * 2 / 1e9, free_b / 1e9);
        return VKLLM_ERR_OK;
    }
    hipStream_t st = ctx->device->stream;
    if (hipMalloc(&fs->tile_slab, total * 2) != hipSuccess || hipMalloc(&fs->xn_t, (size_t)128 * D * 2) != hipSuccess ||
        hipMalloc(&fs->attn_t, (size_t)128 * D * 2) != hipSuccess)
    {
        (void)hipGetLastError();
        free_stream_tiles(fs);
        log_error("short-prompt tiled weights: allocation of %.1f GB failed: prompt steps run on the row-major weights",
                  total * 2 / 1e9);
        return VKLLM_ERR_OK;
    }
    // rows past a step's tokens are read (their outputs are dropped): keep them finite
    HIP_TRY(hipMemsetAsync(fs->xn_t, 0, (size_t)128 * D * 2, st));
    HIP_TRY(hipMemsetAsync(fs->attn_t, 0, (size_t)128 * D * 2, st));
    uint16_t *p = (uint16_t *)fs->tile_slab;
    fs->tiles.resize(mp->L);
    for (uint32_t l = 0; l < mp->L; ++l)
    {
        const ModelPriv::Layer &ly = mp->layers[l];
        FusedState::Tiles &t = fs->tiles[l];
        t.wqkv = p;
        HIP_TRY(vk::launch_tile_weights(st, ly.wqkv, t.wqkv, 3 * D, D, 0));
        p += vk::stream_tiled_elems(3 * D, D, 0);
        t.wo = p;
        HIP_TRY(vk::launch_tile_weights(st, ly.wo, t.wo, D, D, 0));
        p += vk::stream_tiled_elems(D, D, 0);
        t.wug = p;
        HIP_TRY(vk::launch_tile_weights(st, ly.wug, t.wug, 2 * F, D, F));
        p += vk::stream_tiled_elems(2 * F, D, F);
    }
    fs->out_t = p;
    HIP_TRY(vk::launch_tile_weights(st, mp->out_w, fs->out_t, V, D, 0));
    HIP_TRY(hipStreamSynchronize(st));
    fs->stream_ok = true;
    return VKLLM_ERR_OK;
}

static vkllm_err_t ensure_state(vkllm_context *ctx, ModelPriv *mp, uint32_t S)
{
    if (!mp->fs)
    {
        mp->fs = new FusedState();
        FusedState *fs = mp->fs;
        const char *tr = getenv("VKLLM_TRACE_HOST");
        fs->trace = tr && *tr && *tr != '0';
        HIP_TRY(hipMalloc(&fs->step, sizeof(vk::Step)));
        HIP_TRY(hipHostMalloc((void **)&fs->step_h, sizeof(vk::Step), hipHostMallocDefault));
        // read and written by the decode kernels in place: coherent, so no GPU cache holds a stale copy
        HIP_TRY(hipHostMalloc((void **)&fs->dio_slots, 2 * sizeof(vk::DecodeIo), hipHostMallocCoherent));
        memset(fs->dio_slots, 0, 2 * sizeof(vk::DecodeIo));
        fs->dio = fs->dio_slots;
        HIP_TRY(hipMalloc(&fs->slot_ids, 2 * sizeof(uint32_t)));
        HIP_TRY(hipMemset(fs->slot_ids, 0, 2 * sizeof(uint32_t)));
        HIP_TRY(hipMalloc(&fs->slot_logits, (size_t)2 * mp->V * 2));
        for (hipEvent_t &e : fs->slot_done)
            HIP_TRY(hipEventCreateWithFlags(&e, hipEventDisableTiming));
        const char *la = getenv("VKLLM_LAUNCH_AHEAD");
        fs->ahead_enabled = !(la && *la == '0');
        HIP_TRY(hipMalloc(&fs->freqs, sizeof(float) * (mp->hd / 2 + 1)));
        HIP_TRY(hipMemcpyAsync(fs->freqs, mp->rope_freqs.data(), sizeof(float) * mp->hd / 2, hipMemcpyHostToDevice,
                               ctx->device->stream));
        // two-kernel decode attention: chunks of a fixed length of about 256 positions (a multiple of 16), each
        // scored and summed by one block in a single round trip
        const uint32_t cmax = (mp->ctx + 255) / 256;
        fs->att_chunk = ((mp->ctx + cmax - 1) / cmax + 15) / 16 * 16;
        fs->att_cmax = (mp->ctx + fs->att_chunk - 1) / fs->att_chunk;
        const size_t H = mp->H, C = fs->att_cmax;
        const char *sm = getenv("VKLLM_ATTN_SMALL_MAX");
        uint32_t small = sm && *sm ? (uint32_t)strtoul(sm, nullptr, 10) : 1024u;
        vk::AttnDecodeArgs shape{};
        shape.H = mp->H;
        shape.hd = mp->hd;
        shape.ctx = mp->ctx;
        shape.cmax = fs->att_cmax;
        shape.chunk = fs->att_chunk;
        const char *ag = getenv("VKLLM_ATTN_GROUPS");
        fs->attn_max_groups = ag && *ag ? (uint32_t)strtoul(ag, nullptr, 10) : 8u;
        shape.groups = vk::attn_groups(mp->H, mp->hd, fs->attn_max_groups);
        const uint32_t limit = vk::attn_small_limit(shape);
        small = small < limit ? small : limit;
        small = small < kSmallBucket * kSmallBuckets ? small : kSmallBucket * kSmallBuckets;
        fs->attn_small_max = small < mp->ctx ? small : mp->ctx;
        const char *ao = getenv("VKLLM_ATTN_O");
        fs->attn_o = ao && *ao == '1';
        const char *qa = getenv("VKLLM_QKV_ATTN");
        fs->qkv_attn = qa && *qa == '1' && mp->H <= vk::kAttnTailMaxHeads && mp->hd % 8 == 0 &&
                       mp->hd >= 32 && 64 % (mp->hd / 8) == 0;
        HIP_TRY(hipMalloc(&fs->head_count, (size_t)mp->H * sizeof(uint32_t)));
        HIP_TRY(hipMemset(fs->head_count, 0, (size_t)mp->H * sizeof(uint32_t)));
        const char *pe = getenv("VKLLM_PERSIST");
        fs->persist = pe && *pe == '1';
        {
            std::vector<vk::PersistLayer> pl(mp->L);
            for (uint32_t l = 0; l < mp->L; ++l)
            {
                const ModelPriv::Layer &ly = mp->layers[l];
                pl[l] = {ly.wqkv, ly.wo, ly.wug, ly.wd, ly.attn_norm, ly.ffn_norm, ly.kc, ly.vc};
            }
            HIP_TRY(hipMalloc(&fs->persist_layers, pl.size() * sizeof(vk::PersistLayer)));
            HIP_TRY(hipMemcpy(fs->persist_layers, pl.data(), pl.size() * sizeof(vk::PersistLayer),
                              hipMemcpyHostToDevice));
            fs->p_hstride = (mp->D + 127) / 128 * 128;
            fs->p_fstride = (mp->F + 127) / 128 * 128;
            HIP_TRY(hipMalloc(&fs->p_hs, (size_t)(2 * mp->L + 1) * fs->p_hstride * 2));
            HIP_TRY(hipMalloc(&fs->p_qs, (size_t)mp->L * fs->p_hstride * 2));
            HIP_TRY(hipMalloc(&fs->p_attns, (size_t)mp->L * fs->p_hstride * 2));
            HIP_TRY(hipMalloc(&fs->p_acts, (size_t)mp->L * fs->p_fstride * 2));
            HIP_TRY(hipMalloc(&fs->persist_sync, vk::kPersistSyncWords * sizeof(uint32_t)));
            HIP_TRY(hipMemset(fs->persist_sync, 0, vk::kPersistSyncWords * sizeof(uint32_t)));
        }
        const char *al = getenv("VKLLM_ATTN_LONG");
        // head_dim 256 (or chunks shorter than head_dim) takes the two-kernel attention past the short-cache bound
        fs->attn_long = !(al && *al == '0') && vk::attn_long_ok(shape);
        const char *re = getenv("VKLLM_ROPE_EPI");
        fs->rope_epi = !(re && *re == '0');
        const char *ne = getenv("VKLLM_NORM_EPI");
        fs->norm_epi = !(ne && *ne == '0');
        const char *sl = getenv("VKLLM_SPIN_LIMIT");
        if (sl && *sl)
            fs->long_spin_limit = fs->attn_o_spin_limit = (uint32_t)strtoul(sl, nullptr, 10);
        HIP_TRY(hipMalloc(&fs->att_scores, H * mp->ctx * sizeof(float)));
        HIP_TRY(hipMalloc(&fs->att_stats, H * C * 2 * sizeof(float)));
        HIP_TRY(hipMalloc(&fs->att_part, H * C * mp->hd * sizeof(float)));
        HIP_TRY(hipMalloc(&fs->att_count, H * sizeof(uint32_t)));
        HIP_TRY(hipMemset(fs->att_count, 0, H * sizeof(uint32_t)));
        HIP_TRY(hipMalloc(&fs->attn_sync, vk::kAttnSyncWords * sizeof(uint32_t)));
        HIP_TRY(hipMemset(fs->attn_sync, 0, vk::kAttnSyncWords * sizeof(uint32_t)));
        HIP_TRY(hipMalloc(&fs->att_long_sync, H * vk::kAttnLongStride * sizeof(uint32_t)));
        HIP_TRY(hipMemset(fs->att_long_sync, 0, H * vk::kAttnLongStride * sizeof(uint32_t)));
        HIP_TRY(hipMalloc(&fs->gemm_work, kGemmWorkElems * sizeof(float)));
        const char *am = getenv("VKLLM_ARGMAX_EPI");
        fs->argmax_epi = !(am && *am == '0');
        HIP_TRY(hipMalloc(&fs->am_val, kArgmaxCandidates * sizeof(float)));
        HIP_TRY(hipMalloc(&fs->am_idx, kArgmaxCandidates * sizeof(uint32_t)));
        HIP_TRY(hipMalloc(&fs->am_count, vk::kArgmaxSyncWords * sizeof(uint32_t)));
        HIP_TRY(hipMemset(fs->am_count, 0, vk::kArgmaxSyncWords * sizeof(uint32_t)));
        make_node_records(fs, mp->L);
    }
    if (S > 1 && S <= 128 && !mp->fs->stream_tried)
        _CHECK(build_stream_tiles(ctx, mp));
    FusedState *fs = mp->fs;
    if (S <= fs->cap_S)
        return VKLLM_ERR_OK;
    // growing the activation buffers moves them: the captured decode graphs refer to the old ones
    HIP_TRY(hipStreamSynchronize(ctx->device->stream));
    fs->ahead_live = false;
    fs->last_logits = nullptr;
    drop_graphs(fs);
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
    HIP_TRY(hipMalloc(&fs->rope_cs, Sz * mp->hd * sizeof(float)));
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

// One launch of the decode step's kernel family `kid` (KID_F_*) for layer l. The embedding and the residual GEMVs
// write the residual stream in place, or into `resid_out` when it is given (repeatable timing launches).
static hipError_t launch_decode_kernel(vkllm_context *ctx, ModelPriv *mp, KernelId kid, uint32_t l,
                                       uint16_t *resid_out = nullptr)
{
    FusedState *fs = mp->fs;
    hipStream_t st = ctx->device->stream;
    const int cu = ctx->device->cu_count;
    const uint32_t D = mp->D, F = mp->F, V = mp->V, hd = mp->hd;
    const ModelPriv::Layer &ly = mp->layers[l];
    vk::GemvArgs g{};
    g.eps = mp->eps;
    g.K = D;
    switch (kid)
    {
    case KID_F_EMBED:
        return vk::launch_embed_decode(st, fs->dio, fs->step, mp->embd, resid_out ? resid_out : fs->h, V, D,
                                       mp->pad_id, fs->slot_ids + (1 - fs->slot));
    case KID_F_QKV:
        // RMSNorm(h) -> [Wq;Wk;Wv] -> RoPE(q, k); q to fs->q, k and v into the caches at the step's position
        g.x = fs->h;
        g.norm_w = ly.attn_norm;
        g.w = ly.wqkv;
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
        if (fs->qkv_attn_now)
        {
            // and each head's attention by the workgroup that completes the head's rows
            g.attn_out = fs->attn;
            g.head_count = fs->head_count;
            g.H = mp->H;
            g.attn_scale = 1.0f / sqrtf((float)hd);
            g.attn_err = &fs->dio->err;
            return vk::launch_gemv(st, vk::EPI_QKV_ATTN, g, cu);
        }
        return vk::launch_gemv(st, vk::EPI_QKV, g, cu);
    case KID_F_ATTN_SCORES:
    case KID_F_ATTN_PV:
    case KID_F_ATTN_SMALL:
    case KID_F_ATTN_O:
    case KID_F_ATTN_LONG:
    {
        vk::AttnDecodeArgs at{};
        at.q = fs->q;
        at.kc = ly.kc;
        at.vc = ly.vc;
        at.out = fs->attn;
        at.step = fs->step;
        at.scores = fs->att_scores;
        at.stats = fs->att_stats;
        at.part = fs->att_part;
        at.count = fs->att_count;
        at.H = mp->H;
        at.hd = hd;
        at.ctx = mp->ctx;
        at.cmax = fs->att_cmax;
        at.chunk = fs->att_chunk;
        at.groups = vk::attn_groups(mp->H, hd, fs->attn_max_groups);
        at.scale = 1.0f / sqrtf((float)hd);
        at.long_sync = fs->att_long_sync;
        at.err = &fs->dio->err;
        at.spin_limit = kid == KID_F_ATTN_O ? fs->attn_o_spin_limit : fs->long_spin_limit;
        if (kid == KID_F_ATTN_LONG)
            return vk::launch_attn_long(st, at, cu);
        if (kid == KID_F_ATTN_SMALL)
            return vk::launch_attn_small(st, at, fs->small_kv_max);
        if (kid == KID_F_ATTN_O)
        {
            // attention, then h + Wo attn in the same launch
            vk::AttnOArgs ao{};
            ao.at = at;
            ao.wo = ly.wo;
            ao.resid = fs->h;
            ao.out = resid_out ? resid_out : fs->h;
            ao.sync = fs->attn_sync;
            ao.err = &fs->dio->err;
            return vk::launch_attn_o(st, ao, fs->small_kv_max, cu);
        }
        return kid == KID_F_ATTN_SCORES ? vk::launch_attn_scores(st, at) : vk::launch_attn_pv(st, at);
    }
    case KID_F_O_RESID:
    case KID_F_DOWN_RESID:
        // h + W x, x the attention output (Wo) or up * silu(gate) (Wd)
        g.x = kid == KID_F_O_RESID ? fs->attn : fs->act;
        g.w = kid == KID_F_O_RESID ? ly.wo : ly.wd;
        g.K = kid == KID_F_O_RESID ? D : F;
        g.rows = D;
        g.units = (D + 1) / 2;
        g.out = resid_out ? resid_out : fs->h;
        g.resid = fs->h;
        return vk::launch_gemv(st, vk::EPI_RESID, g, cu);
    case KID_F_GATEUP:
        // RMSNorm(h) -> [Wu;Wg] -> up * silu(gate) into fs->act
        g.x = fs->h;
        g.norm_w = ly.ffn_norm;
        g.w = ly.wug;
        g.rows = 2 * F;
        g.units = F;
        g.out = fs->act;
        return vk::launch_gemv(st, vk::EPI_GATEUP, g, cu);
    case KID_F_LOGITS:
        g.x = fs->h;
        g.norm_w = mp->out_norm;
        g.w = mp->out_w;
        g.rows = V;
        g.units = (V + 1) / 2;
        g.out = fs->slot_logits + (size_t)fs->slot * V;
        if (!fs->argmax_epi)
            return vk::launch_gemv(st, vk::EPI_PLAIN, g, cu);
        // the logits and their arg max (what KID_F_ARGMAX computes) in one launch
        g.am_ids = fs->slot_ids + fs->slot;
        g.am_io = fs->dio;
        g.am_val = fs->am_val;
        g.am_idx = fs->am_idx;
        g.am_count = fs->am_count;
        g.am_cap = kArgmaxCandidates;
        return vk::launch_gemv(st, vk::EPI_ARGMAX, g, cu);
    case KID_F_ARGMAX:
        return vk::launch_argmax_rows(st, fs->slot_logits + (size_t)fs->slot * V, fs->slot_ids + fs->slot, 1, V,
                                      fs->dio);
    default:
        return hipErrorInvalidValue;
    }
}

// the node a single-token step's launch of family kid is charged to
static void charge_decode(vkllm_context *ctx, FusedState *fs, KernelId kid, uint32_t l)
{
    switch (kid)
    {
    case KID_F_EMBED:
        return charge(ctx, fs, NS_EMBEDDED);
    case KID_F_QKV:
        return charge(ctx, fs, NS_Q, l);
    case KID_F_ATTN_SMALL:
    case KID_F_ATTN_LONG:
    case KID_F_ATTN_SCORES:
    case KID_F_ATTN_O:
        return charge(ctx, fs, NS_SCORES, l);
    case KID_F_ATTN_PV:
        return charge(ctx, fs, NS_ATTN, l);
    case KID_F_O_RESID:
        return charge(ctx, fs, NS_WO, l);
    case KID_F_GATEUP:
        return charge(ctx, fs, NS_UP, l);
    case KID_F_DOWN_RESID:
        return charge(ctx, fs, NS_DOWN, l);
    case KID_F_LOGITS:
        return charge(ctx, fs, NS_LOGITS);
    case KID_F_ARGMAX:
        return charge(ctx, fs, NS_OUTPUT);
    default:
        return;
    }
}

#define DTRY(_ctx, _mp, _kid, _l)                                                                                   \
    do                                                                                                              \
    {                                                                                                               \
        charge_decode((_ctx), (_mp)->fs, (_kid), (_l));                                                             \
        KTRY(_ctx, _kid, launch_decode_kernel((_ctx), (_mp), (_kid), (_l)));                                        \
    } while (0)

// the attention variant of a single-token step at cache length kv: the short-cache bucket b < kSmallBuckets, or
// kSmallBuckets for the long-cache path
static uint32_t decode_variant(const FusedState *fs, uint32_t kv)
{
    return kv <= fs->attn_small_max ? (kv - 1) / kSmallBucket : kSmallBuckets;
}

// The persistent step after the embedding (its input row, fs->p_hs[0]) for the current slot and short-cache bound
static hipError_t launch_persist(vkllm_context *ctx, ModelPriv *mp)
{
    FusedState *fs = mp->fs;
    vk::PersistArgs pa{};
    pa.layers = fs->persist_layers;
    pa.L = mp->L;
    pa.D = mp->D;
    pa.F = mp->F;
    pa.V = mp->V;
    pa.H = mp->H;
    pa.hd = mp->hd;
    pa.ctx = mp->ctx;
    pa.eps = mp->eps;
    pa.scale = 1.0f / sqrtf((float)mp->hd);
    pa.step = fs->step;
    pa.freqs = fs->freqs;
    pa.out_norm = mp->out_norm;
    pa.out_w = mp->out_w;
    pa.hs = fs->p_hs;
    pa.qs = fs->p_qs;
    pa.attns = fs->p_attns;
    pa.acts = fs->p_acts;
    pa.hstride = fs->p_hstride;
    pa.fstride = fs->p_fstride;
    pa.logits = fs->slot_logits + (size_t)fs->slot * mp->V;
    pa.small_max = fs->small_kv_max;
    pa.sync = fs->persist_sync;
    pa.err = &fs->dio->err;
    pa.spin_limit = fs->attn_o_spin_limit;
    pa.am_ids = fs->slot_ids + fs->slot;
    pa.am_io = fs->dio;
    pa.am_val = fs->am_val;
    pa.am_idx = fs->am_idx;
    pa.am_count = fs->am_count;
    pa.am_cap = kArgmaxCandidates;
    return vk::launch_decode_persist(ctx->device->stream, pa, ctx->device->cu_count);
}

// decode: S == 1, position from fs->step; `variant` (decode_variant) picks the attention kernels and, for short caches,
// the positions bound of their launches
static vkllm_err_t enqueue_decode(vkllm_context *ctx, ModelPriv *mp, uint32_t variant)
{
    const bool small_attn = variant < kSmallBuckets;
    if (small_attn)
    {
        const uint32_t end = (variant + 1) * kSmallBucket;
        mp->fs->small_kv_max = end < mp->fs->attn_small_max ? end : mp->fs->attn_small_max;
    }
    if (small_attn && mp->fs->persist && !ctx->device->timing)
    {
        // the embedding row, then every layer and the vocabulary product in one launch
        FusedState *fs = mp->fs;
        KTRY(ctx, KID_F_EMBED,
             vk::launch_embed_decode(ctx->device->stream, fs->dio, fs->step, mp->embd, fs->p_hs, mp->V, mp->D,
                                     mp->pad_id, fs->slot_ids + (1 - fs->slot)));
        const hipError_t e = launch_persist(ctx, mp);
        fs->p_variant[variant] = e == hipSuccess;
        if (e == hipSuccess)
            return VKLLM_ERR_OK;
        if (e == hipErrorInvalidConfiguration) // the device does not hold the grid: separate kernels from now on
            fs->persist = false;
        else if (e != hipErrorInvalidValue) // (a shape or positions bound the launch does not take: this bucket)
            return hip_fail(e, "launch_decode_persist", __FILE__, __LINE__);
    }
    // caches of at most kAttnTailMaxKv positions (this bucket's end): the attention in the QKV product's launch
    const bool tail_attn = small_attn && mp->fs->qkv_attn && mp->fs->small_kv_max <= vk::kAttnTailMaxKv;
    mp->fs->qkv_attn_now = tail_attn;
    DTRY(ctx, mp, KID_F_EMBED, 0);
    for (uint32_t l = 0; l < mp->L; ++l)
    {
        DTRY(ctx, mp, KID_F_QKV, l);
        if (tail_attn)
        {
            DTRY(ctx, mp, KID_F_O_RESID, l);
            DTRY(ctx, mp, KID_F_GATEUP, l);
            DTRY(ctx, mp, KID_F_DOWN_RESID, l);
            continue;
        }
        bool fused_o = false;
        if (small_attn && mp->fs->attn_o)
        {
            charge_decode(ctx, mp->fs, KID_F_ATTN_O, l);
            const hipError_t e = timed(ctx, pipeline_of(ctx, KID_F_ATTN_O),
                                       [&]() { return launch_decode_kernel(ctx, mp, KID_F_ATTN_O, l); });
            if (e == hipSuccess)
                fused_o = true;
            else if (e == hipErrorInvalidConfiguration) // not enough room for both parts: two launches from now on
                mp->fs->attn_o = false;
            else
                return hip_fail(e, "launch_attn_o", __FILE__, __LINE__);
        }
        if (!fused_o)
        {
            bool long_done = false;
            if (!small_attn && mp->fs->attn_long)
            {
                charge_decode(ctx, mp->fs, KID_F_ATTN_LONG, l);
                const hipError_t e = timed(ctx, pipeline_of(ctx, KID_F_ATTN_LONG),
                                           [&]() { return launch_decode_kernel(ctx, mp, KID_F_ATTN_LONG, l); });
                if (e == hipSuccess)
                    long_done = true;
                else if (e == hipErrorInvalidConfiguration) // the chunk blocks do not fit at once: two kernels
                    mp->fs->attn_long = false;
                else
                    return hip_fail(e, "launch_attn_long", __FILE__, __LINE__);
            }
            if (small_attn)
                DTRY(ctx, mp, KID_F_ATTN_SMALL, l);
            else if (!long_done)
            {
                DTRY(ctx, mp, KID_F_ATTN_SCORES, l);
                DTRY(ctx, mp, KID_F_ATTN_PV, l);
            }
            DTRY(ctx, mp, KID_F_O_RESID, l);
        }
        DTRY(ctx, mp, KID_F_GATEUP, l);
        DTRY(ctx, mp, KID_F_DOWN_RESID, l);
    }
    if (mp->fs->argmax_epi)
    {
        charge_decode(ctx, mp->fs, KID_F_LOGITS, 0);
        const hipError_t e =
            timed(ctx, pipeline_of(ctx, KID_F_LOGITS), [&]() { return launch_decode_kernel(ctx, mp, KID_F_LOGITS, 0); });
        if (e == hipSuccess)
            return VKLLM_ERR_OK;
        if (e != hipErrorInvalidValue)
            return hip_fail(e, "logits + arg max", __FILE__, __LINE__);
        // the vocabulary product's shape does not take the arg-max epilogue (nothing was launched): two kernels
        mp->fs->argmax_epi = false;
    }
    DTRY(ctx, mp, KID_F_LOGITS, 0);
    DTRY(ctx, mp, KID_F_ARGMAX, 0);
    return VKLLM_ERR_OK;
}

// A short-prompt product streamed from its tiled weights; a STREAM_PARTIAL product then goes through the split-K
// reduce with `reduce_epi` (GEMM_QKV_ROPE with `rope`, or GEMM_RESID into C with `norm`). STREAM_QKV_ROPE takes
// `rope` itself.
static hipError_t stream_product(hipStream_t st, FusedState *fs, int epi, const uint16_t *X, const uint16_t *Wt,
                                 uint16_t *C, uint32_t M, uint32_t N, uint32_t K, uint32_t ldc, int reduce_epi = -1,
                                 const vk::GemmRope *rope = nullptr, const vk::GemmNorm *norm = nullptr)
{
    uint32_t splits = 0;
    hipError_t e =
        vk::launch_stream_gemm(st, epi, X, Wt, C, fs->gemm_work, kGemmWorkElems, M, N, K, ldc, &splits, rope);
    if (e != hipSuccess || epi != vk::STREAM_PARTIAL)
        return e;
    return vk::launch_gemm_reduce(st, reduce_epi, fs->gemm_work, C, M, N, splits, rope, norm);
}

static vkllm_err_t enqueue_prefill(vkllm_context *ctx, ModelPriv *mp, uint32_t S, uint32_t offset)
{
    FusedState *fs = mp->fs;
    hipStream_t st = ctx->device->stream;
    const int cu = ctx->device->cu_count;
    const uint32_t D = mp->D, F = mp->F, V = mp->V, hd = mp->hd;
    const float scale = 1.0f / sqrtf((float)hd);
    charge(ctx, fs, NS_EMBEDDED);
    KTRY(ctx, KID_F_EMBED, vk::launch_embed_rows(st, fs->toks, S, mp->embd, fs->h, V, D, mp->pad_id));
    // RoPE in the QKV product's epilogue where the shape allows it (angles computed once for all layers);
    // otherwise the product is stored and a separate kernel rotates and appends
    const bool rope_epi = fs->rope_epi && D % 64 == 0 && hd >= 32 && (hd & (hd - 1)) == 0;
    if (rope_epi)
    {
        charge(ctx, fs, NS_RK, 0);
        KTRY(ctx, KID_F_ROPE_KV, vk::launch_rope_table(st, fs->rope_cs, fs->freqs, offset, S, hd));
    }
    // every residual product also leaves the next RMSNorm of the residual stream in xn (in the split-K reduce when
    // K is split, else as a separate pass)
    // prompts of at most 128 tokens: the QKV, output, gate/up and vocabulary products stream their tiled weights,
    // reading fragment-ordered activations (the normalised rows in xn_t, the attention output in attn_t)
    const bool streamed = fs->stream_ok && S <= 128 && rope_epi && fs->norm_epi;
    uint16_t *xn = streamed ? fs->xn_t : fs->xn;
    // the streamed vocabulary product stores 4 logits of a row as one 8-byte vector, so its rows of V must stay
    // 8-byte aligned; otherwise the tile GEMM takes the logits, and the last norm writes its row-major input
    const bool stream_logits = streamed && V % 4 == 0;
    uint16_t *attn = streamed ? fs->attn_t : fs->attn;
    charge(ctx, fs, NS_ATTN_NORM, 0);
    KTRY(ctx, KID_F_RMSNORM, vk::launch_rmsnorm_rows(st, fs->h, mp->layers[0].attn_norm, xn, S, D, mp->eps, streamed));
    for (uint32_t l = 0; l < mp->L; ++l)
    {
        const ModelPriv::Layer &ly = mp->layers[l];
        if (streamed)
        {
            const vk::GemmRope rope{fs->q, ly.kc, ly.vc, fs->rope_cs, offset, D, hd, mp->ctx};
            charge(ctx, fs, NS_Q, l);
            // above 32 tokens the product splits the tokens and rotates in its own epilogue; shorter prompts split K
            // and rotate in the reduce
            if (S > 32)
                KTRY(ctx, KID_F_GEMM, stream_product(st, fs, vk::STREAM_QKV_ROPE, xn, fs->tiles[l].wqkv, nullptr, S, 3 * D, D, 0, -1, &rope));
            else
                KTRY(ctx, KID_F_GEMM, stream_product(st, fs, vk::STREAM_PARTIAL, xn, fs->tiles[l].wqkv, fs->qkv, S, 3 * D, D, 3 * D, vk::GEMM_QKV_ROPE, &rope));
        }
        else if (rope_epi)
        {
            const vk::GemmRope rope{fs->q, ly.kc, ly.vc, fs->rope_cs, offset, D, hd, mp->ctx};
            charge(ctx, fs, NS_Q, l);
            KTRY(ctx, KID_F_GEMM, vk::launch_gemm(st, vk::GEMM_QKV_ROPE, fs->xn, ly.wqkv, fs->qkv, S, 3 * D, D, 3 * D, 0, cu, fs->gemm_work, kGemmWorkElems, &rope));
        }
        else
        {
            charge(ctx, fs, NS_Q, l);
            KTRY(ctx, KID_F_GEMM, vk::launch_gemm(st, vk::GEMM_PLAIN, fs->xn, ly.wqkv, fs->qkv, S, 3 * D, D, 3 * D, 0, cu, fs->gemm_work, kGemmWorkElems));
            charge(ctx, fs, NS_RQ, l);
            KTRY(ctx, KID_F_ROPE_KV,
                 vk::launch_rope_kv(st, fs->qkv, fs->q, ly.kc, ly.vc, fs->freqs, offset, S, D, hd, mp->ctx));
        }
        charge(ctx, fs, NS_SCORES, l);
        KTRY(ctx, KID_F_ATTN_PREFILL,
             vk::launch_attn_prefill(st, fs->q, ly.kc, ly.vc, attn, offset, S, mp->H, hd, mp->ctx, scale, streamed));
        const vk::GemmNorm ffn_norm{ly.ffn_norm, xn, mp->eps, streamed};
        charge(ctx, fs, NS_WO, l);
        if (streamed)
            KTRY(ctx, KID_F_GEMM, stream_product(st, fs, vk::STREAM_PARTIAL, attn, fs->tiles[l].wo, fs->h, S, D, D, D, vk::GEMM_RESID, nullptr, &ffn_norm));
        else
            KTRY(ctx, KID_F_GEMM, vk::launch_gemm(st, vk::GEMM_RESID, fs->attn, ly.wo, fs->h, S, D, D, D, 0, cu, fs->gemm_work, kGemmWorkElems, nullptr, fs->norm_epi ? &ffn_norm : nullptr));
        if (!fs->norm_epi)
        {
            charge(ctx, fs, NS_FFN_NORM, l);
            KTRY(ctx, KID_F_RMSNORM, vk::launch_rmsnorm_rows(st, fs->h, ly.ffn_norm, fs->xn, S, D, mp->eps));
        }
        // SwiGLU in the product's epilogue where the shape allows it (gate and up rows read as interleaved blocks);
        // otherwise up and SiLU(gate) are stored side by side and multiplied by a separate kernel
        charge(ctx, fs, NS_UP, l);
        if (streamed)
            KTRY(ctx, KID_F_GEMM, stream_product(st, fs, vk::STREAM_SWIGLU, xn, fs->tiles[l].wug, fs->act, S, 2 * F, D, F));
        else if (D % 64 == 0 && F % 32 == 0)
            KTRY(ctx, KID_F_GEMM,
                 vk::launch_gemm(st, vk::GEMM_SWIGLU, fs->xn, ly.wug, fs->act, S, 2 * F, D, F, F, cu, fs->gemm_work, kGemmWorkElems));
        else
        {
            KTRY(ctx, KID_F_GEMM,
                 vk::launch_gemm(st, vk::GEMM_SILU_HI, fs->xn, ly.wug, fs->ug, S, 2 * F, D, 2 * F, F, cu, fs->gemm_work, kGemmWorkElems));
            charge(ctx, fs, NS_MUL, l);
            KTRY(ctx, KID_F_SWIGLU, vk::launch_swiglu(st, fs->ug, fs->act, S, F));
        }
        const bool last = l + 1 == mp->L;
        const vk::GemmNorm next_norm{last ? mp->out_norm : mp->layers[l + 1].attn_norm,
                                     last && !stream_logits ? fs->xn : xn, mp->eps, last ? stream_logits : streamed};
        charge(ctx, fs, NS_DOWN, l);
        KTRY(ctx, KID_F_GEMM, vk::launch_gemm(st, vk::GEMM_RESID, fs->act, ly.wd, fs->h, S, D, F, D, 0, cu, fs->gemm_work, kGemmWorkElems, nullptr, fs->norm_epi ? &next_norm : nullptr));
        if (!fs->norm_epi)
        {
            if (l + 1 < mp->L)
                charge(ctx, fs, NS_ATTN_NORM, l + 1);
            else
                charge(ctx, fs, NS_OUTPUT_NORM);
            KTRY(ctx, KID_F_RMSNORM, vk::launch_rmsnorm_rows(st, fs->h, next_norm.w, fs->xn, S, D, mp->eps));
        }
    }
    charge(ctx, fs, NS_LOGITS);
    if (stream_logits)
        KTRY(ctx, KID_F_GEMM, stream_product(st, fs, vk::STREAM_PLAIN, xn, fs->out_t, fs->logits, S, V, D, V));
    else
        KTRY(ctx, KID_F_GEMM, vk::launch_gemm(st, vk::GEMM_PLAIN, fs->xn, mp->out_w, fs->logits, S, V, D, V, 0, cu, fs->gemm_work, kGemmWorkElems));
    charge(ctx, fs, NS_OUTPUT);
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
    if (p->S > 1 && (size_t)(p->offset + p->S) * sizeof(float) > 60 * 1024)
    {
        log_error("prefill attention holds %u scores per row in LDS; at most %u", p->offset + p->S,
                  (unsigned)(60 * 1024 / sizeof(float)));
        return VKLLM_ERR_ARGS;
    }
    return ensure_state(ctx, mp, p->S);
}

// the slot whose DecodeIo, logits row and arg-max id the decode launches being enqueued use
static void select_slot(FusedState *fs, int k)
{
    fs->slot = k;
    fs->dio = fs->dio_slots + k;
}

// Drops a step launched ahead (after it finished) and points the decode launches at the last completed step's
// slot and inputs: for work on the stream that must not be mistaken for, or run with, that step.
static vkllm_err_t discard_ahead(vkllm_context *ctx, FusedState *fs)
{
    HIP_TRY(hipStreamSynchronize(ctx->device->stream));
    fs->ahead_live = false;
    select_slot(fs, fs->done_slot);
    fs->dio->offset = fs->done_offset;
    fs->dio->token = fs->done_token;
    fs->dio->token_dev = 0;
    fs->dio->err = 0;
    return VKLLM_ERR_OK;
}

vkllm_err_t fused_plan_discard_ahead(vkllm_context *ctx, vkllm_graph *graph)
{
    auto *p = (FusedPlan *)graph->plan;
    ModelPriv *mp = p ? model_priv(p->model) : nullptr;
    if (!mp || !mp->fs)
        return VKLLM_ERR_OK;
    return discard_ahead(ctx, mp->fs);
}

// Enqueues one single-token step: a replay of the captured graph for this attention variant (captured on first
// use), or direct launches when graph replay or timing says so.
static vkllm_err_t launch_decode_step(vkllm_context *ctx, ModelPriv *mp, uint32_t v)
{
    FusedState *fs = mp->fs;
    hipStream_t st = ctx->device->stream;
    if (!ctx->device->graph_replay || ctx->device->timing)
        return enqueue_decode(ctx, mp, v);
    const int k = fs->slot;
    if (!fs->exec[k][v])
    {
        HIP_TRY(hipStreamBeginCapture(st, hipStreamCaptureModeRelaxed));
        vkllm_err_t rc = enqueue_decode(ctx, mp, v);
        hipGraph_t g = nullptr;
        hipError_t ce = hipStreamEndCapture(st, &g);
        if (rc != VKLLM_ERR_OK)
        {
            if (g)
                (void)hipGraphDestroy(g);
            return rc;
        }
        HIP_TRY(ce);
        fs->graph[k][v] = g;
        HIP_TRY(hipGraphInstantiate(&fs->exec[k][v], g, nullptr, nullptr, 0));
    }
    HIP_TRY(hipGraphLaunch(fs->exec[k][v], st));
    fs->last_exec = v;
    fs->last_exec_slot = k;
    return VKLLM_ERR_OK;
}

// Timing mode: the step's node records start from zero (pending launches of earlier work are read first)
static vkllm_err_t reset_node_costs(vkllm_context *ctx, FusedState *fs)
{
    if (!ctx->device->timing)
        return VKLLM_ERR_OK;
    HIP_TRY(timing_flush(ctx));
    for (vkllm_pipeline &r : fs->node_pipes)
        r.last_ns = 0;
    return VKLLM_ERR_OK;
}

// Timing mode, after the step: each graph node whose record received launches points at it, so
// vkllm_pipeline_query_exec_time(node->pipeline) gives the node's share of the step, as the reference's per-node
// timestamps do (tests/vkllm_test_infer_gguf.c:205-225). The records sum to the step's kernel time.
static vkllm_err_t attach_node_costs(vkllm_context *ctx, FusedState *fs, vkllm_graph *graph)
{
    if (!ctx->device->timing)
        return VKLLM_ERR_OK;
    HIP_TRY(timing_flush(ctx));
    for (size_t i = 0; i < graph->nodes->used_n; ++i)
    {
        vkllm_tensor *t = graph->nodes->data[i];
        auto it = fs->node_index.find(t->name);
        if (it != fs->node_index.end() && fs->node_pipes[it->second].last_ns > 0)
            t->pipeline = &fs->node_pipes[it->second];
    }
    return VKLLM_ERR_OK;
}

vkllm_err_t fused_plan_run(vkllm_context *ctx, vkllm_graph *graph)
{
    auto *p = (FusedPlan *)graph->plan;
    ModelPriv *mp = model_priv(p->model);
    _CHECK(fused_plan_init(ctx, graph));
    FusedState *fs = mp->fs;
    _CHECK(reset_node_costs(ctx, fs));
    hipStream_t st = ctx->device->stream;
    const uint32_t S = p->S;
    // the step's ids are in the mapped input tensor's host mirror (written by vkllm_commands_upload)
    const uint32_t *toks = (const uint32_t *)p->input_toks->data.host;
    vkllm_tensor *out = graph->output_node;
    if (S == 1)
    {
        // position and token go through the slot's pinned block that the step's first kernel reads; the arg max
        // writes the chosen id back into it
        const uint64_t t0 = fs->trace ? host_ns() : 0;
        const bool direct = !ctx->device->graph_replay || ctx->device->timing;
        const uint32_t variant = decode_variant(fs, p->offset + 1);
        int slot;
        if (fs->ahead_live && !direct && fs->ahead_offset == p->offset && fs->ahead_token == toks[0])
            slot = fs->ahead_slot; // launched ahead with this very token at this position: queued or done
        else
        {
            // a step launched ahead for another token or position runs before this one (stream order); this step
            // rewrites the cache rows it wrote, or never reads them
            slot = fs->ahead_live ? 1 - fs->ahead_slot : 1 - fs->done_slot;
            select_slot(fs, slot);
            fs->dio->offset = p->offset;
            fs->dio->token = toks[0];
            fs->dio->token_dev = 0;
            fs->dio->err = 0;
            _CHECK(launch_decode_step(ctx, mp, variant));
            HIP_TRY(hipEventRecord(fs->slot_done[slot], st));
        }
        fs->ahead_live = false;
        if (fs->ahead_enabled && !direct && p->offset + 1 < mp->ctx)
        {
            // the step at p + 1 behind this one, its token this step's device-side arg max
            const int nx = 1 - slot;
            select_slot(fs, nx);
            fs->dio->offset = p->offset + 1;
            fs->dio->token = 0;
            fs->dio->token_dev = 1;
            fs->dio->err = 0;
            _CHECK(launch_decode_step(ctx, mp, decode_variant(fs, p->offset + 2)));
            HIP_TRY(hipEventRecord(fs->slot_done[nx], st));
            fs->ahead_live = true;
            fs->ahead_slot = nx;
            fs->ahead_offset = p->offset + 1;
        }
        select_slot(fs, slot);
        const uint64_t t1 = fs->trace ? host_ns() : 0;
        HIP_TRY(hipEventSynchronize(fs->slot_done[slot]));
        if (((volatile vk::DecodeIo *)fs->dio)->err)
        {
            // A bounded wait between workgroups gave up (the GPU is shared or busy, so not every block of the launch
            // was resident). Let the step launched ahead finish and drop it, clear the counters the launches left,
            // switch to the attention kernels that never wait, and run the step again: it starts from the
            // embedding and rewrites the same cache rows, so a second run gives the step's result.
            log_error("decode step at position %u: a kernel's wait for other workgroups gave up; running it again "
                      "with attention kernels that do not wait",
                      p->offset);
            HIP_TRY(hipStreamSynchronize(st));
            fs->ahead_live = false;
            HIP_TRY(hipMemsetAsync(fs->attn_sync, 0, vk::kAttnSyncWords * sizeof(uint32_t), st));
            HIP_TRY(hipMemsetAsync(fs->att_long_sync, 0, (size_t)mp->H * vk::kAttnLongStride * sizeof(uint32_t), st));
            HIP_TRY(hipMemsetAsync(fs->att_count, 0, (size_t)mp->H * sizeof(uint32_t), st));
            HIP_TRY(hipMemsetAsync(fs->persist_sync, 0, vk::kPersistSyncWords * sizeof(uint32_t), st));
            drop_graphs(fs);
            fs->attn_long = false;
            fs->attn_o = false;
            fs->persist = false;
            fs->dio->offset = p->offset;
            fs->dio->token = toks[0];
            fs->dio->token_dev = 0;
            fs->dio->err = 0;
            _CHECK(launch_decode_step(ctx, mp, variant));
            HIP_TRY(hipStreamSynchronize(st));
            if (((volatile vk::DecodeIo *)fs->dio)->err)
                return VKLLM_ERR_VULKAN;
        }
        const uint32_t id = ((volatile vk::DecodeIo *)fs->dio)->id;
        fs->io_h[0] = id;
        if (fs->ahead_live)
            fs->ahead_token = id;
        fs->done_slot = slot;
        fs->done_offset = p->offset;
        fs->done_token = toks[0];
        fs->last_logits = fs->slot_logits + (size_t)slot * mp->V;
        if (fs->trace)
        {
            fs->trace_steps += 1;
            fs->trace_enqueue_ns += t1 - t0;
            fs->trace_wait_ns += host_ns() - t1;
        }
    }
    else
    {
        fs->ahead_live = false; // a step launched ahead runs first (stream order); nothing reads what it wrote
        fs->step_h->offset = p->offset;
        fs->step_h->S = S;
        memcpy(fs->io_h, toks, (size_t)S * 4);
        HIP_TRY(hipMemcpyAsync(fs->step, fs->step_h, sizeof(vk::Step), hipMemcpyHostToDevice, st));
        HIP_TRY(hipMemcpyAsync(fs->toks, fs->io_h, (size_t)S * 4, hipMemcpyHostToDevice, st));
        _CHECK(enqueue_prefill(ctx, mp, S, p->offset));
        HIP_TRY(hipMemcpyAsync(fs->io_h, fs->ids, (size_t)S * 4, hipMemcpyDeviceToHost, st));
        HIP_TRY(hipStreamSynchronize(st));
        fs->last_logits = fs->logits;
    }
    p->ran = true;
    // results: the arg-max ids into the output node, as the reference's mapped ARG_MAX output holds them
    if (out->data.host)
    {
        memcpy(out->data.host, fs->io_h, (size_t)S * 4);
        out->data.host_current = true;
        out->data.valid = false;
        return attach_node_costs(ctx, fs, graph);
    }
    void *out_dev = tensor_dev(ctx, out);
    if (!out_dev)
        return VKLLM_ERR_ALLOC;
    HIP_TRY(hipMemcpyAsync(out_dev, S == 1 ? fs->slot_ids + fs->done_slot : fs->ids, (size_t)S * 4,
                           hipMemcpyDeviceToDevice, st));
    HIP_TRY(hipStreamSynchronize(st));
    out->data.valid = true;
    return attach_node_costs(ctx, fs, graph);
}

// ---- extension: fused-step internals for tests and measurement ----

// Copies the fp16 logits of the last fused step ([S, vocab]) into `dst`.
extern "C" vkllm_err_t vkllm_hip_model_last_logits(struct vkllm_context *ctx, struct vkllm_models_llama2 *model,
                                                   uint16_t *dst, uint32_t rows)
{
    DeviceScope device_scope(ctx);
    _CHECK_ARGS(ctx && model && dst);
    ModelPriv *mp = model_priv(model);
    _CHECK_ARGS(mp && mp->fs && mp->fs->logits && rows <= mp->fs->cap_S);
    // a single-token step's logits are in its slot's row (a step launched ahead writes the other slot's)
    const uint16_t *src = mp->fs->last_logits ? mp->fs->last_logits : mp->fs->logits;
    _CHECK_ARGS(src == mp->fs->logits || rows == 1);
    HIP_TRY(hipMemcpyAsync(dst, src, (size_t)rows * mp->V * 2, hipMemcpyDeviceToHost, ctx->device->stream));
    HIP_TRY(hipStreamSynchronize(ctx->device->stream));
    return VKLLM_ERR_OK;
}

extern "C" vkllm_err_t vkllm_hip_model_time_kernel(struct vkllm_context *ctx, struct vkllm_models_llama2 *model,
                                                   const char *family, uint32_t reps, uint64_t *total_ns)
{
    DeviceScope device_scope(ctx);
    _CHECK_ARGS(ctx && model && family && reps > 0 && total_ns);
    ModelPriv *mp = model_priv(model);
    _CHECK_ARGS(mp && mp->fs && mp->fs->cap_S >= 1 && mp->fs->h);
    FusedState *fs = mp->fs;
    static const struct
    {
        const char *name;
        KernelId kid;
    } families[] = {{"fused_embed", KID_F_EMBED},         {"fused_qkv_rope", KID_F_QKV},
                    {"fused_attn_scores", KID_F_ATTN_SCORES}, {"fused_attn_pv", KID_F_ATTN_PV},
                    {"fused_attn_small", KID_F_ATTN_SMALL}, {"fused_attn_o", KID_F_ATTN_O},
                    {"fused_attn_long", KID_F_ATTN_LONG},
                    {"fused_o_resid", KID_F_O_RESID},     {"fused_gateup", KID_F_GATEUP},
                    {"fused_down_resid", KID_F_DOWN_RESID}, {"fused_logits", KID_F_LOGITS},
                    {"fused_argmax", KID_F_ARGMAX}};
    // the launches below recompute the last completed step (same token, same position): a step launched ahead is
    // dropped first, so that nothing is mistaken for it
    _CHECK(discard_ahead(ctx, fs));
    const bool whole = strcmp(family, "decode_step") == 0, persist = strcmp(family, "decode_persist") == 0;
    int kid = -1;
    for (const auto &f : families)
        if (strcmp(family, f.name) == 0)
            kid = f.kid;
    _CHECK_ARGS(whole || persist || kid >= 0);
    const int replay = (int)decode_variant(fs, fs->done_offset + 1);
    if (whole && (fs->last_exec < 0 || !fs->exec[fs->done_slot][replay]))
    {
        log_error("decode_step timing needs a captured decode step (graph replay on, one single-token step run)");
        return VKLLM_ERR_ARGS;
    }
    if ((kid == KID_F_ATTN_SMALL || kid == KID_F_ATTN_O) && fs->dio->offset + 1 > fs->attn_small_max)
    {
        log_error("%s takes at most %u positions; the last step had %u", family, fs->attn_small_max,
                  fs->dio->offset + 1);
        return VKLLM_ERR_ARGS;
    }
    {
        // the launches of the last step's bucket
        const uint32_t b = decode_variant(fs, fs->dio->offset + 1);
        if (b < kSmallBuckets)
        {
            const uint32_t end = (b + 1) * kSmallBucket;
            fs->small_kv_max = end < fs->attn_small_max ? end : fs->attn_small_max;
        }
        fs->qkv_attn_now = b < kSmallBuckets && fs->qkv_attn && fs->small_kv_max <= vk::kAttnTailMaxKv;
        if (persist && (b >= kSmallBuckets || !fs->persist || !fs->p_variant[b]))
        {
            log_error("decode_persist timing needs a last single-token step that ran as the persistent launch");
            return VKLLM_ERR_ARGS;
        }
    }
    hipStream_t st = ctx->device->stream;
    // the residual GEMVs write into fs->xn (a scratch row) so that repeating them leaves the model state unchanged
    auto launch = [&](uint32_t r) -> hipError_t {
        if (whole)
            return hipGraphLaunch(fs->exec[fs->done_slot][replay], st);
        if (persist) // the last step again from its embedding row (same token and position: same cache rows)
            return launch_persist(ctx, mp);
        return launch_decode_kernel(ctx, mp, (KernelId)kid, r % mp->L, fs->xn);
    };
    if (persist) // the last step's embedding row and position again (a step launched ahead wrote its own)
        HIP_TRY(vk::launch_embed_decode(st, fs->dio, fs->step, mp->embd, fs->p_hs, mp->V, mp->D, mp->pad_id,
                                        fs->slot_ids + (1 - fs->slot)));
    // one untimed launch so the first timed one does not pay for code loading
    HIP_TRY(launch(0));
    hipEvent_t ev[2];
    HIP_TRY(hipEventCreate(&ev[0]));
    if (hipEventCreate(&ev[1]) != hipSuccess)
    {
        (void)hipEventDestroy(ev[0]);
        return VKLLM_ERR_VULKAN;
    }
    hipError_t e = hipEventRecord(ev[0], st);
    for (uint32_t r = 0; r < reps && e == hipSuccess; ++r)
        e = launch(r + 1);
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

extern "C" vkllm_err_t vkllm_hip_gemm_streamed(struct vkllm_context *ctx, int epi, const uint16_t *A,
                                               const uint16_t *B, uint16_t *C, uint32_t M, uint32_t N, uint32_t K,
                                               uint32_t ldc, uint32_t splits)
{
    DeviceScope device_scope(ctx);
    _CHECK_ARGS(ctx && A && B && C && M > 0 && M <= 128 && N > 0 && K >= 16 && K % 16 == 0 && splits <= 8);
    _CHECK_ARGS(epi == vk::GEMM_PLAIN || epi == vk::GEMM_RESID || epi == vk::GEMM_SWIGLU);
    _CHECK_ARGS(epi == vk::GEMM_PLAIN ? ldc >= N : (epi == vk::GEMM_RESID ? ldc == N && N % 32 == 0 : N % 32 == 0 && ldc >= N / 2));
    _CHECK_ARGS(((uintptr_t)A | (uintptr_t)B) % 16 == 0 && (uintptr_t)C % 8 == 0 && ldc % 4 == 0);
    hipStream_t st = ctx->device->stream;
    const uint32_t F = epi == vk::GEMM_SWIGLU ? N / 2 : 0;
    const size_t xt_elems = (size_t)128 * K, wt_elems = vk::stream_tiled_elems(N, K, F);
    const size_t work_elems = epi == vk::GEMM_RESID ? (size_t)8 * M * N : 0;
    uint16_t *xt = nullptr, *wt = nullptr;
    float *work = nullptr;
    hipError_t e = hipMalloc(&xt, xt_elems * 2);
    if (e == hipSuccess)
        e = hipMalloc(&wt, wt_elems * 2);
    if (e == hipSuccess && work_elems)
        e = hipMalloc(&work, work_elems * sizeof(float));
    if (e == hipSuccess)
        e = vk::launch_tile_activations(st, A, xt, M, K);
    if (e == hipSuccess)
        e = vk::launch_tile_weights(st, B, wt, N, K, F);
    if (e == hipSuccess)
    {
        const int sepi = epi == vk::GEMM_PLAIN ? vk::STREAM_PLAIN
                                                : (epi == vk::GEMM_RESID ? vk::STREAM_PARTIAL : vk::STREAM_SWIGLU);
        e = timed(ctx, pipeline_of(ctx, KID_F_GEMM), [&]() {
            uint32_t n_splits = splits;
            hipError_t r = vk::launch_stream_gemm(st, sepi, xt, wt, C, work, work_elems, M, N, K, ldc, &n_splits);
            if (r != hipSuccess || sepi != vk::STREAM_PARTIAL)
                return r;
            return vk::launch_gemm_reduce(st, vk::GEMM_RESID, work, C, M, N, n_splits);
        });
    }
    if (e == hipSuccess)
        e = hipStreamSynchronize(st);
    (void)hipFree(xt);
    (void)hipFree(wt);
    (void)hipFree(work);
    if (e != hipSuccess)
        return hip_fail(e, "vkllm_hip_gemm_streamed", __FILE__, __LINE__);
    return VKLLM_ERR_OK;
}

extern "C" vkllm_err_t vkllm_hip_gemm(struct vkllm_context *ctx, int epi, const uint16_t *A, const uint16_t *B,
                                      uint16_t *C, uint32_t M, uint32_t N, uint32_t K, uint32_t ldc, uint32_t split,
                                      float *work, uint64_t work_elems)
{
    DeviceScope device_scope(ctx);
    _CHECK_ARGS(ctx && A && B && C && M > 0 && N > 0 && K >= 8 && K % 8 == 0);
    _CHECK_ARGS(epi == vk::GEMM_PLAIN || epi == vk::GEMM_SILU_HI || epi == vk::GEMM_RESID || epi == vk::GEMM_SWIGLU);
    _CHECK_ARGS(epi == vk::GEMM_SWIGLU ? (K % 64 == 0 && N % 64 == 0 && split * 2 == N && ldc >= split && ldc % 8 == 0)
                                       : ldc >= N);
    _CHECK_ARGS(work != nullptr || work_elems == 0);
    // the tiles read A, B and the split-K partials as 16-byte vectors; the SwiGLU reduce stores C as 16-byte vectors
    _CHECK_ARGS(((uintptr_t)A | (uintptr_t)B | (uintptr_t)work) % 16 == 0);
    _CHECK_ARGS(epi != vk::GEMM_SWIGLU || (uintptr_t)C % 16 == 0);
    hipStream_t st = ctx->device->stream;
    KTRY(ctx, KID_F_GEMM,
         vk::launch_gemm(st, epi, A, B, C, M, N, K, ldc, split, ctx->device->cu_count, work, (size_t)work_elems));
    HIP_TRY(hipStreamSynchronize(st));
    return VKLLM_ERR_OK;
}
