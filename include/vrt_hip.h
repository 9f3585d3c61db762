/*
 * vrt_hip.h -- C ABI of the MI355X (gfx950) HIP implementation of Vortex-RT's Gemma 3
 * Q8_0 token loop. Plain pointers and sizes only; every function returns VRT_OK (0) or a
 * nonzero status whose message is available from vrt_last_error() on the calling thread.
 *
 * Each declaration names the reference interface it replaces. The reference exposes a
 * C++ class API (namespace vortexrt) over Vulkan; the headers under include/vortexrt keep that
 * C++ surface, implemented on top of these functions in libvortexrt.so.
 *
 * Conventions
 *  - Device pointers come from vrt_alloc (or any HIP allocation on the context's device).
 *  - Kernel entry points are stream-ordered on the context's single stream; vrt_sync()
 *    gives the reference's synchronous semantics (every reference run* call blocks on a
 *    fence, src/q8_matvec.cpp:1321-1350). vrt_memcpy is synchronous.
 *  - Argument validation mirrors the reference's and happens on the host before any
 *    launch, so an invalid call never reaches the GPU.
 *  - A context or executor handle must not be used from two threads at once.
 */
#ifndef VRT_HIP_H
#define VRT_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define VRT_OK 0
#define VRT_ERR_INVALID 1   /* argument check failed (the reference throws std::runtime_error) */
#define VRT_ERR_HIP 2       /* HIP runtime error */
#define VRT_ERR_STATE 3     /* executor state: non-contiguous position, context exceeded, ... */
#define VRT_ERR_NUMERIC 4   /* non-finite hidden state, softmax failure, invalid argmax */

typedef struct vrt_ctx vrt_ctx;
typedef struct vrt_g3 vrt_g3;

/* include/vortexrt/argmax.hpp:12-17 (ArgmaxResult, 8 bytes). */
typedef struct vrt_argmax_result {
    uint32_t index;
    float value;
} vrt_argmax_result;

/* include/vortexrt/vulkan_context.hpp:13-32 (DeviceCapabilities), HIP fields. */
typedef struct vrt_device_info {
    char name[256];
    char arch[64];
    uint32_t device_index;
    uint32_t vendor_id;
    uint32_t device_id;
    uint32_t subgroup_size;       /* wavefront size: 64 */
    uint32_t compute_units;
    uint32_t fp16, int8, storage8, storage16;
    uint64_t device_local_bytes;
    uint64_t l2_bytes;
} vrt_device_info;

/* Thread-local message of the last failing call on this thread. */
const char* vrt_last_error(void);

/* ---- context and memory ------------------------------------------------------------ */

/* VulkanContext(std::string device_selector), include/vortexrt/vulkan_context.hpp:45 and
 * src/vulkan_context.cpp:116-317: selector is "" (then env VORTEXRT_DEVICE, then device 0),
 * a decimal index, or a case-insensitive substring of the device name. */
int vrt_ctx_create(const char* selector, vrt_ctx** out);
int vrt_ctx_destroy(vrt_ctx* ctx);
/* VulkanContext::capabilities(), include/vortexrt/vulkan_context.hpp:56. */
int vrt_ctx_info(const vrt_ctx* ctx, vrt_device_info* out);

#define VRT_MEM_DEVICE 0      /* VK_MEMORY_PROPERTY_DEVICE_LOCAL_BIT -> hipMalloc */
#define VRT_MEM_HOST 1        /* HOST_VISIBLE | HOST_COHERENT -> pinned hipHostMalloc */

/* Buffer(ctx, size, usage, memory_properties), include/vortexrt/buffer.hpp:13-17. The
 * allocation is zero-filled and rounded up to 256 bytes plus 256 bytes of slack. */
int vrt_alloc(vrt_ctx* ctx, uint64_t bytes, uint32_t kind, void** out);
int vrt_free(vrt_ctx* ctx, void* ptr);
/* Buffer::upload / Buffer::download, include/vortexrt/buffer.hpp:32-33: synchronous copy
 * between any two addresses (host or device). */
int vrt_memcpy(vrt_ctx* ctx, void* dst, const void* src, uint64_t bytes);
int vrt_memset(vrt_ctx* ctx, void* dst, int value, uint64_t bytes);
/* Waits for all work on the context's stream (the reference's vkWaitForFences). */
int vrt_sync(vrt_ctx* ctx);
/* The hipStream_t every kernel of this context is launched on. */
int vrt_stream(vrt_ctx* ctx, void** stream);

/* Timing on the context's stream (hipEvent pairs). */
int vrt_event_create(vrt_ctx* ctx, void** ev);
int vrt_event_record(vrt_ctx* ctx, void* ev);
int vrt_event_elapsed_ms(void* start, void* stop, float* ms);
int vrt_event_destroy(void* ev);

/* ---- Q8_0 kernels ------------------------------------------------------------------- */
/* Weights are GGUF Q8_0: rows of input_dim/32 blocks of 34 bytes {f16 scale LE, int8[32]}.
 * weight_byte_offset must be 4-byte aligned and input_dim a nonzero multiple of 32
 * (src/q8_matvec.cpp:801-820). weights_bytes is the readable size at `weights`. */

/* Q8MatVecPipeline::run, include/vortexrt/q8_matvec.hpp:35-41: y = W x. */
int vrt_q8_matvec(vrt_ctx* ctx, const void* weights, uint64_t weights_bytes, uint32_t weight_byte_offset,
                  const float* x, float* y, uint32_t input_dim, uint32_t output_dim);

/* Q8MatVecPipeline::run_staged_pair / run_staged_triplet, include/vortexrt/q8_matvec.hpp:
 * 74-100: n (1..8) matrices sharing x, outputs packed contiguously in call order. */
int vrt_q8_matvec_multi(vrt_ctx* ctx, const void* weights, uint64_t weights_bytes, uint32_t n,
                        const uint32_t* weight_byte_offsets, const uint32_t* output_dims,
                        uint32_t input_dim, const float* x, float* y_packed);

/* Q8MatVecPipeline::run_staged_ffn, include/vortexrt/q8_matvec.hpp:57-72 and
 * src/q8_matvec.cpp:1360-2004: gate = Wg x, up = Wu x, h = gelu_tanh(gate) * up,
 * y = Wd h. Two launches: gate/up with the GELU product as its epilogue, then down.
 * workspace (2 * ffn_dim floats) ends up holding [h | up], the gate half holding h as in
 * the reference's workspace. */
int vrt_q8_ffn(vrt_ctx* ctx, const void* weights, uint64_t weights_bytes,
               uint32_t gate_offset, uint32_t up_offset, uint32_t down_offset,
               uint32_t input_dim, uint32_t ffn_dim, uint32_t output_dim,
               const float* x, float* workspace, uint64_t workspace_bytes, float* y);

/* No counterpart in the reference. vrt_q8_ffn without a workspace argument, for callers that
 * cannot allocate device memory (code under stream capture, serving loops, harnesses that forbid
 * hipMalloc): the [h | up] workspace is a static per-device array of the library (128 KiB), so
 * the call allocates nothing. ffn_dim <= 16384, else VRT_ERR_INVALID. Every call on a device
 * shares that device's array: calls on one device that overlap (two contexts, two streams) race. */
int vrt_q8_ffn_noalloc(vrt_ctx* ctx, const void* weights, uint64_t weights_bytes,
                       uint32_t gate_offset, uint32_t up_offset, uint32_t down_offset,
                       uint32_t input_dim, uint32_t ffn_dim, uint32_t output_dim,
                       const float* x, float* y);

/* shaders/gelu_mul.comp: gate[i] = gelu_tanh(gate[i]) * up[i]. */
int vrt_gelu_mul(vrt_ctx* ctx, float* gate, const float* up, uint32_t n);

/* ArgmaxPipeline::run, include/vortexrt/argmax.hpp:29-32 and shaders/argmax.comp:
 * NaN never wins, larger wins, equal values -> lower index. out is device-visible. */
int vrt_argmax(vrt_ctx* ctx, const float* x, uint32_t n, vrt_argmax_result* out);

/* Quantiser of record (src/q8_test_main.cpp:18-131; variant 1 = src/ffn_test_main.cpp:
 * 112-215) on the GPU, bit-exact: n floats (multiple of 32) -> n/32 blocks. */
int vrt_q8_quantize(vrt_ctx* ctx, const float* x, uint64_t n, uint32_t variant, void* out_blocks);

/* GgufFile::read_q8_0_row dequant (src/gguf.cpp:620-635) on the GPU: n_blocks -> floats. */
int vrt_q8_dequantize(vrt_ctx* ctx, const void* blocks, uint64_t n_blocks, float* out);

/* ---- Gemma 3 executor --------------------------------------------------------------- */

/* Gemma3Config, include/vortexrt/gemma3.hpp:19-33. */
typedef struct vrt_g3_config {
    uint32_t context_length;
    uint32_t embedding_length;
    uint32_t block_count;
    uint32_t feed_forward_length;
    uint32_t head_count;
    uint32_t head_count_kv;
    uint32_t head_dim;
    uint32_t value_dim;
    uint32_t vocab_size;
    uint32_t sliding_window;
    float rms_epsilon;
    float global_rope_base;
    float local_rope_base;
} vrt_g3_config;

/* Per-block tensors (src/gemma3.cpp:456-505): Q8_0 byte offsets into the arena and host
 * pointers to the F32 norm weights (copied to the device by vrt_g3_create). */
typedef struct vrt_g3_layer {
    uint64_t attn_q, attn_k, attn_v, attn_output, ffn_gate, ffn_up, ffn_down;
    const float* attn_norm;             /* [embedding_length] */
    const float* attn_q_norm;           /* [head_dim] */
    const float* attn_k_norm;           /* [head_dim] */
    const float* post_attention_norm;   /* [embedding_length] */
    const float* ffn_norm;              /* [embedding_length] */
    const float* post_ffw_norm;         /* [embedding_length] */
} vrt_g3_layer;

typedef struct vrt_g3_desc {
    vrt_g3_config config;
    const void* arena;          /* device copy of the GGUF tensor-data section (caller-owned) */
    uint64_t arena_bytes;
    uint64_t token_embd;        /* byte offset of token_embd.weight (tied LM head) */
    const float* output_norm;   /* host [embedding_length] */
    const vrt_g3_layer* layers; /* [block_count] */
    uint32_t eos_token_id;      /* tokenizer.ggml.eos_token_id (src/gemma3.cpp:443-446) */
} vrt_g3_desc;

/* Device half of the Gemma3Model constructor (src/gemma3.cpp:510-654): KV cache, RoPE
 * tables (src/gemma3.cpp:1309-1369 evaluated on the host), norm weights, workspaces and
 * the captured decode-step graph. Shapes are validated as the reference does
 * (src/gemma3.cpp:219-257). */
int vrt_g3_create(vrt_ctx* ctx, const vrt_g3_desc* desc, vrt_g3** out);
/* Fails with VRT_ERR_STATE, destroying nothing, while a vrt_g3_batch created over this executor
 * is alive: destroy batches first, then the executor, then the context. */
int vrt_g3_destroy(vrt_g3* g3);

/* Gemma3Model::reset_cache, src/gemma3.cpp:1454-1460. */
int vrt_g3_reset(vrt_g3* g3);

/* Gemma3Model::decode_token, src/gemma3.cpp:1462-1882. top_k == 0 skips the LM head;
 * top_k >= 1 runs the tied LM head fused with greedy argmax (result in *out); top_k > 1
 * also keeps the logits for vrt_g3_logits. hidden_out (embedding_length floats, host) may
 * be NULL. On any error the KV cache is reset, as in the reference. */
int vrt_g3_decode(vrt_g3* g3, uint32_t token, uint32_t position, uint32_t top_k,
                  vrt_argmax_result* out, float* hidden_out);

/* Batched prompt prefill (the prompt loop of src/gemma3.cpp:2099-2111 in one pass; the
 * reference has no batched path): resets the cache, then runs positions 0..n-1 with every
 * projection as a Q8_0 x activation GEMM on MFMA and causal local/global attention; the last
 * position runs the LM head as vrt_g3_decode would with top_k (0 skips it, 1 is the fused
 * argmax into *out, > 1 keeps the logits for vrt_g3_logits). hidden_out (embedding_length
 * floats, host) may be NULL. Decoding continues at position n. Prompts longer than the
 * batched workspace (min(context_length, 2048) positions) run as consecutive segments of that
 * many positions, each attending to the earlier ones through the KV cache; shapes the batched
 * kernels do not cover run as serial decode steps. On any error the KV cache is reset. */
int vrt_g3_prefill(vrt_g3* g3, const uint32_t* tokens, uint32_t n, uint32_t top_k, vrt_argmax_result* out,
                   float* hidden_out);

/* Logits of the last step that ran the LM head with top_k > 1 (host copy, n floats). */
int vrt_g3_logits(vrt_g3* g3, float* host_logits, uint32_t n);

/* Gemma3Model::generate_greedy_tokens, src/gemma3.cpp:2080-2149: the whole loop runs on
 * the device (graph replays, the next token chosen on the device) with one host sync.
 * out_tokens holds up to max_new ids; generation stops after EOS as in the reference. */
int vrt_g3_generate(vrt_g3* g3, const uint32_t* prompt, uint32_t n_prompt, uint32_t max_new,
                    uint32_t* out_tokens, uint32_t* n_out);

/* The same loop split for callers that overlap or time it: vrt_g3_start resets and uploads
 * the prompt; vrt_g3_step enqueues n steps (asynchronous, stream-ordered; n_prompt +
 * max_new - 1 steps in total complete the generation); vrt_g3_collect waits and returns the
 * generated ids (stopping after EOS) as vrt_g3_generate does. */
int vrt_g3_start(vrt_g3* g3, const uint32_t* prompt, uint32_t n_prompt, uint32_t max_new);
int vrt_g3_step(vrt_g3* g3, uint32_t n);
int vrt_g3_collect(vrt_g3* g3, uint32_t* out_tokens, uint32_t* n_out);

/* Teacher-forced run (validation): resets, then step i consumes tokens[i] at position i;
 * steps i >= first_logit_step run the LM head and record their greedy result in out[i]. */
int vrt_g3_forced(vrt_g3* g3, const uint32_t* tokens, uint32_t n, uint32_t first_logit_step,
                  vrt_argmax_result* out);

/* Executor options. The persistent kernel (one cooperative launch runs a batch of steps) is
 * used when the device and shape support it; otherwise, or with VRT_G3_OPT_PERSISTENT = 0,
 * each step is the multi-kernel sequence, replayed from a hipGraph unless
 * VRT_G3_OPT_USE_GRAPH = 0. VRT_G3_OPT_QUERY_PERSISTENT returns VRT_OK when the persistent
 * kernel is available (value ignored). When the device refuses its cooperative launch (on
 * ROCm while another live process has made one on the same GPU) the executor continues on the
 * multi-kernel path and the query reports the refusal. */
#define VRT_G3_OPT_USE_GRAPH 1
#define VRT_G3_OPT_PERSISTENT 2
#define VRT_G3_OPT_QUERY_PERSISTENT 3
#define VRT_G3_OPT_TRACE 4          /* 1: timestamp the phases of the first step of each launch */
/* 1: the KV cache holds fp16 keys and values (IEEE round to nearest even of the fp32 k and v
 * after QK-norm and RoPE; every position's attention, the current one's included, uses the
 * rounded values), 2 bytes per element instead of 4. Switching resets the cache. The
 * reference's README lists an fp16/bf16 KV cache as its next residency step
 * (README.md:190-192); it has no implementation to follow. */
#define VRT_G3_OPT_KV_F16 5
/* 1: the KV cache holds bfloat16 keys and values (IEEE round to nearest even of the fp32 k and
 * v, as for KV_F16; 8 exponent bits, 7 mantissa bits), 2 bytes per element. KV_F16 and KV_BF16
 * select one format: setting either to 1 replaces the other, setting the one in use to 0
 * returns to fp32. Switching resets the cache. Same roadmap item (README.md:190-192). */
#define VRT_G3_OPT_KV_BF16 12
/* 1 (default): decode steps at short histories run on the phase-team persistent kernel (four
 * teams of workgroups, each running one phase type of every block, with one-way hand-offs); later
 * positions, or all with 0, run on the all-workgroup persistent kernel. Both give the same
 * results to the stated tolerances. VRT_G3_OPT_QUERY_TEAM returns VRT_OK when the team kernel
 * is available for the shape and device (value ignored). VRT_G3_OPT_QUERY_TEAM_POSITIONS (read
 * with vrt_g3_get_option) gives the position below which steps run on the team kernel (0 when it
 * is unavailable): the context length at the shapes it is built for, where histories longer
 * than a workgroup holds on chip (136 positions of fp32 KV entries at the Gemma-3-270M shape, 208
 * of 16-bit ones) split into chunks per head. No reference counterpart. */
#define VRT_G3_OPT_TEAM 6
#define VRT_G3_OPT_QUERY_TEAM 7
/* Projection fusion and the Q8 lane policy (Gemma3Model::set_projection_fusion_enabled and the
 * q8_lane_override of its constructor, src/gemma3.cpp:94-172, :656-671). FUSION 1 (default): the
 * fused sequence (the persistent kernels, or on the multi-kernel path one q|k|v launch and one
 * gate/up launch with the GELU product in its epilogue, as run_q8_triplet / the fused FFN);
 * 0: every step runs the multi-kernel sequence with q, k, v, gate and up as launches of their
 * own and the GELU product as a launch after them (:1529-1541, :1783-1847). Q8_LANES 0
 * (default): row slots sized per matrix; 8, 16, 32 or 64: the projections' rows run in slots of
 * that many lanes on the multi-kernel path (a 2048-input row needs at least 16), like the
 * reference's forced narrow pipeline; other values fail as the reference's constructor does.
 * Both change only the schedule: results agree to the stated tolerances. Either setting drops
 * the captured step graph. QUERY_Q8_LANES (read with vrt_g3_get_option) gives the lanes per row
 * the embedding-width projections run with. */
#define VRT_G3_OPT_FUSION 8
#define VRT_G3_OPT_Q8_LANES 9
#define VRT_G3_OPT_QUERY_Q8_LANES 10
#define VRT_G3_OPT_QUERY_TEAM_POSITIONS 11
/* Read with vrt_g3_get_option: the position from which team-kernel steps run its chunked
 * variant (histories split across a head's workgroups); equal to QUERY_TEAM_POSITIONS when the
 * shape has none. Each variant is its own launch. */
#define VRT_G3_OPT_QUERY_TEAM_CHUNKED 13

/* Phase trace of the last persistent launch (tracing tool; no reference counterpart, which
 * only has CLI wall timers, src/gemma_main.cpp:194-232): out[w * slots + k] is the
 * s_memrealtime tick (100 MHz) at which workgroup w finished phase k of the launch's first
 * step: k = 0 step start, 5l + 1 .. 5l + 5 phases A..E of block l, 5L + 1 end of the blocks,
 * 5L + 2 end of the LM head. Entries of phases a workgroup does not run keep older values.
 * When the last launch ran the team kernel (VRT_G3_OPT_TEAM), slots = 2L + 3: k < L the time
 * workgroup w's team had the inputs of its phase of block k, L + k the time it had published
 * it, 2L step start, 2L + 1 the LM head's final norm done, 2L + 2 LM head done (0: not run).
 * Workgroup w belongs to team (w % 8) / 2 (0 q|k|v, 1 attention + O, 2 gate/up, 3 down). */
int vrt_g3_read_trace(vrt_g3* g3, uint64_t* out, uint64_t cap, uint32_t* nwg, uint32_t* slots);

/* Raw tagged words {fp32 bits | tag << 32} of a persistent-kernel exchange buffer as the last
 * launch left them (diagnostics; no reference counterpart): which = 0 q|k|v, 1 attention chunk
 * partials, 2 attention output projection, 3 gelu(gate)*up, 4 down projection, 5 argmax
 * partials. *n receives the word count; synchronises the context's stream. */
int vrt_g3_read_exchange(vrt_g3* g3, uint32_t which, uint64_t* out, uint64_t cap, uint64_t* n);
int vrt_g3_set_option(vrt_g3* g3, uint32_t option, uint32_t value);
/* Current value of an executor option: USE_GRAPH, PERSISTENT, TEAM, KV_F16, KV_BF16, FUSION and Q8_LANES
 * as last set, QUERY_Q8_LANES, QUERY_TEAM_POSITIONS and QUERY_TEAM_CHUNKED as described above (the getters projection_fusion_enabled and
 * narrow_q8_lane_count of include/vortexrt/gemma3.hpp read these). */
int vrt_g3_get_option(vrt_g3* g3, uint32_t option, uint32_t* value);

/* Batched greedy decode: up to max_seqs independent sequences share the executor's weights, each
 * with its own KV cache of max_ctx positions (<= context_length). The reference decodes one
 * sequence (src/gemma3.cpp:1462-1882, one KV cache per model); batching is its roadmap's
 * "continuous batching" (README.md:190-193), with no implementation to follow. A step advances
 * n sequences by one position each: sequence seqs[i] consumes tokens[i] at its next position
 * (a prompt token or the token it generated last) and results[i] receives its greedy next token
 * and logit (all arrays on the host, n <= max_seqs, distinct ids). Every projection and the
 * LM head are GEMMs over the n rows on MFMA (the numerics of vrt_g3_prefill), attention runs
 * per sequence over its own cache. On any error every sequence of the step is reset to
 * position 0, as the reference resets its cache. */
typedef struct vrt_g3_batch vrt_g3_batch;
int vrt_g3_batch_create(vrt_g3* g3, uint32_t max_seqs, uint32_t max_ctx, vrt_g3_batch** out);
/* The batch reads its executor's weights and launches on its context's stream: destroy it
 * before the executor (vrt_g3_destroy refuses while it is alive). */
int vrt_g3_batch_destroy(vrt_g3_batch* b);
/* Sequence seq (or every sequence, seq = 0xffffffff) restarts at position 0. */
int vrt_g3_batch_reset(vrt_g3_batch* b, uint32_t seq);
int vrt_g3_batch_step(vrt_g3_batch* b, const uint32_t* seqs, const uint32_t* tokens, uint32_t n,
                      vrt_argmax_result* results);
/* Next position of sequence seq. */
int vrt_g3_batch_position(vrt_g3_batch* b, uint32_t seq, uint32_t* pos);
/* Logits of row `row` (< n) of the last step (host copy, n floats <= vocab_size). */
int vrt_g3_batch_logits(vrt_g3_batch* b, uint32_t row, float* host_logits, uint32_t n);

/* Launches the tied LM head + argmax kernel `iters` times back to back between two
 * hipEvents on the context stream (current hidden state) and reports the mean duration. */
int vrt_g3_time_lm_head(vrt_g3* g3, uint32_t iters, float* mean_us);

#ifdef __cplusplus
}
#endif
#endif
