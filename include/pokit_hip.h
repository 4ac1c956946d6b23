/*
 * pokit_hip.h -- C ABI of the PokitLMs MI355X (gfx950) HIP backend for the
 * routed-MoE K-quant path.
 *
 * Conventions follow the reference C API (include/pokitlms/pokitlms.h of
 * RemydreScarlet/PokitLMs v0.4.0): opaque handles, a status enum whose values
 * 0-4 match pokitlms_status (pokitlms.h:18-24), error text truncated and
 * NUL-terminated into a caller buffer (src/c_api.cpp:22-27), no exceptions
 * across the ABI.  Host buffers are caller-owned; device memory is owned by
 * the context.  Calls on one context must be serialized (the reference
 * backends serialize with a mutex, src/vulkan_linear.cpp:635; C handles
 * require serialized calls, pokitlms.h:81).
 *
 * GGUF type ids: F32 0, F16 1, Q4_0 2, Q4_1 3, Q5_0 6, Q5_1 7, Q8_0 8, Q2_K 10,
 * Q3_K 11, Q4_K 12, Q5_K 13, Q6_K 14, BF16 30 (src/gguf_reader.cpp:21-57).  Matrices are GGUF [in, out] tensors:
 * `out` rows of `in` elements, each row a run of encoded blocks.  Expert
 * tensors are [in, out, n_experts] with the expert index slowest, so expert e
 * is the contiguous slice e * (out * row_bytes) (src/expert_store.cpp:17-36).
 */
#ifndef POKIT_HIP_H
#define POKIT_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define PK_HIP_VERSION_MAJOR 0
#define PK_HIP_VERSION_MINOR 1
#define PK_HIP_VERSION_PATCH 0

typedef enum pk_hip_status {
    PK_HIP_STATUS_OK = 0,
    PK_HIP_STATUS_INVALID_ARGUMENT = 1,
    PK_HIP_STATUS_RUNTIME_ERROR = 2,
    PK_HIP_STATUS_BUFFER_TOO_SMALL = 3,
    PK_HIP_STATUS_INTERNAL_ERROR = 4,
    /* The backend does not cover this type/shape: the caller runs its CPU
     * kernel, exactly as TensorLinearBackend::try_linear returning false
     * (include/pokitlms/model/tensor_linear.hpp:14-15). */
    PK_HIP_STATUS_UNSUPPORTED = 5
} pk_hip_status;

typedef struct pk_hip_ctx pk_hip_ctx;
typedef struct pk_hip_weight pk_hip_weight;

/* Options of pk_hip_create; zero-initialise, then set struct_size. */
typedef struct pk_hip_options {
    uint32_t struct_size;  /* sizeof(pk_hip_options) */
    /* Non-zero: time every launch with HIP events and accumulate per-kernel
     * device time into pk_hip_stats (synchronises after each call). */
    uint32_t time_kernels;
} pk_hip_options;

/* Counters in the spirit of VulkanLinearStats (include/pokitlms/gpu/
 * vulkan_linear.hpp:41-67) and ExpertCacheStats (qwen3_moe_runner.hpp:44-52). */
typedef struct pk_hip_stats {
    uint64_t matvec_calls;
    uint64_t moe_decode_calls;
    uint64_t dispatches;                /* kernel launches */
    uint64_t q4_0_dispatches, q8_0_dispatches, q4_k_dispatches, q5_k_dispatches,
        q6_k_dispatches, float_dispatches;
    uint64_t weight_bytes;              /* algorithmic weight bytes streamed */
    uint64_t resident_bytes;            /* device bytes held by weight handles */
    uint64_t uploaded_bytes;            /* host->device weight bytes */
    uint64_t router_fallbacks;          /* tokens whose routing needed exact serial logits */
    uint64_t router_candidates;         /* rows recomputed serially, summed */
    uint64_t expert_hits;               /* routed expert accesses (all resident) */
    uint64_t expert_misses;             /* always 0: experts never leave HBM */
    /* Device time in ns; filled when pk_hip_options.time_kernels != 0. */
    uint64_t matvec_ns, router_ns, gate_up_ns, down_ns;
    uint64_t router_launches, gate_up_launches, down_launches, matvec_launches;
    uint64_t prefill_calls, prefill_tokens, prefill_ns;
    uint64_t prefill_route_ns, prefill_gate_up_ns, prefill_down_ns;
    uint64_t q4_1_dispatches;
    uint64_t q5_0_dispatches, q5_1_dispatches, q2_k_dispatches, q3_k_dispatches;
} pk_hip_stats;

const char* pk_hip_version(void);

/* Non-zero when `ggml_type` has a matvec kernel: F32/F16/BF16/Q4_0/Q4_1/
 * Q5_0/Q5_1/Q8_0/Q2_K/Q3_K/Q4_K/Q5_K/Q6_K, every type tensor_linear
 * dispatches (src/tensor_linear.cpp:176-187; the Vulkan backend's list,
 * src/vulkan_linear.cpp:78-83, omits Q5_0/Q5_1/Q2_K/Q3_K). */
int pk_hip_type_supported(uint32_t ggml_type);

/* Backend construction / destruction: VulkanLinearBackend ctor and dtor
 * (src/vulkan_linear.cpp:88-95, 738-758).  device < 0 selects device 0. */
pk_hip_status pk_hip_create(int device, const pk_hip_options* options, pk_hip_ctx** out_ctx,
                            char* error_buffer, size_t error_capacity);
void pk_hip_destroy(pk_hip_ctx* ctx);

/* Writes "<device name> (<gfx arch>, <CUs> CUs, <GiB> GiB)" of the context's
 * device, truncated and NUL-terminated: VulkanLinearBackend::device_name
 * (include/pokitlms/gpu/vulkan_linear.hpp:80). */
pk_hip_status pk_hip_device_name(const pk_hip_ctx* ctx, char* buffer, size_t capacity);

/* Uploads one GGUF tensor [in, out(, n_experts)] to HBM, where it stays
 * resident: the whole-model device cache of the Vulkan backend
 * (src/vulkan_linear.cpp:516-563) and, for expert tensors, the ExpertStore
 * with every expert resident (src/expert_store.cpp:17-36, 81-141).
 * n_experts == 0 means a plain matrix.  nbytes must equal the encoded size. */
pk_hip_status pk_hip_upload(pk_hip_ctx* ctx, uint32_t ggml_type, uint64_t in, uint64_t out,
                            uint32_t n_experts, const void* host_bytes, uint64_t nbytes,
                            pk_hip_weight** out_weight, char* error_buffer,
                            size_t error_capacity);

/* As pk_hip_upload, from device memory the caller owns (device-to-device
 * copy).  The copy starts after all earlier work on the device has finished,
 * so a source still being written on another stream is complete. */
pk_hip_status pk_hip_upload_device(pk_hip_ctx* ctx, uint32_t ggml_type, uint64_t in,
                                   uint64_t out, uint32_t n_experts, const void* device_bytes,
                                   uint64_t nbytes, pk_hip_weight** out_weight,
                                   char* error_buffer, size_t error_capacity);

void pk_hip_weight_release(pk_hip_weight* weight);
uint64_t pk_hip_weight_bytes(const pk_hip_weight* weight);
/* Device address of the resident weight (read-only use by the caller).  Q4_0,
 * Q8_0, Q6_K, Q5_0 and Q3_K are held in a planar layout (each block field in
 * a plane of its own per slice, expert slices 256-byte aligned), the other
 * types in their GGUF encoding; pk_hip_weight_download returns the GGUF
 * bytes of any type. */
const void* pk_hip_weight_device_ptr(const pk_hip_weight* weight);

/* Copies the weight's GGUF encoding (nbytes = the uploaded size) into
 * caller-owned host memory: TensorReader::read_all of the resident tensor
 * (include/pokitlms/model/tensor_reader.hpp:34). */
pk_hip_status pk_hip_weight_download(const pk_hip_weight* weight, void* host_bytes,
                                     uint64_t nbytes, char* error_buffer,
                                     size_t error_capacity);

/* y[b] = W . x[b] for b < batch (1..8): TensorLinearBackend::try_linear
 * (tensor_linear.hpp:16-17; Vulkan: src/vulkan_linear.cpp:612-736), with
 * caller-owned host buffers x [batch][in] and y [batch][out].  expert selects
 * one slice of an expert tensor (UINT32_MAX for a plain matrix).  Returns
 * PK_HIP_STATUS_UNSUPPORTED (CPU fallback) for types or widths without a
 * kernel; shape errors return INVALID_ARGUMENT; device failures return
 * RUNTIME_ERROR and mark the context failed (src/vulkan_linear.cpp:636,731-735). */
pk_hip_status pk_hip_matvec(pk_hip_ctx* ctx, const pk_hip_weight* weight, uint32_t expert,
                            const float* x, uint32_t batch, float* y, char* error_buffer,
                            size_t error_capacity);

/* As pk_hip_matvec with device buffers, enqueued on `stream` (a hipStream_t;
 * NULL = the context stream) without synchronising. */
pk_hip_status pk_hip_matvec_async(pk_hip_ctx* ctx, const pk_hip_weight* weight,
                                  uint32_t expert, const float* device_x, uint32_t batch,
                                  float* device_y, void* stream, char* error_buffer,
                                  size_t error_capacity);

/* y = W . x in the CPU's own summation order: per row ((0 + dot_0) + dot_1)
 * + ... over blocks, each block dot a left-to-right FP32 chain (linear_k,
 * linear_quantized, linear: src/quantized_linear.cpp:360-423,
 * src/linear.cpp:10-31), so outputs equal the reference's bit for bit.
 * Slower than pk_hip_matvec (one serial chain per row and block); used by the
 * reference-order model decode.  F32 and Q4_0/Q4_1/Q8_0/Q4_K/Q5_K/Q6_K, width up
 * to 8192.  Host buffers, batch 1. */
pk_hip_status pk_hip_matvec_reference_order(pk_hip_ctx* ctx, const pk_hip_weight* weight,
                                           uint32_t expert, const float* x, float* y,
                                           char* error_buffer, size_t error_capacity);

/* One Qwen3-MoE routed layer. router: F32 [hidden, n_experts]; gate/up:
 * [hidden, ffn, n_experts]; down: [ffn, hidden, n_experts].  top_k routes by
 * route_experts (src/qwen3_moe_runner.cpp:267-305): expert ids and their
 * order bit-exact; normalize = qwen3moe.expert_weights_norm; scale multiplies
 * every route weight (Qwen3.5 expert_weights_scale,
 * src/qwen35_runner.cpp:738; 1 for Qwen3-MoE). */
typedef struct pk_hip_moe_layer {
    const pk_hip_weight* router;
    const pk_hip_weight* gate;
    const pk_hip_weight* up;
    const pk_hip_weight* down;
    uint32_t top_k;
    uint32_t normalize;
    float scale;
} pk_hip_moe_layer;

/* MoE block for one token (src/qwen3_moe_runner.cpp:644-691): x is the
 * normalised hidden state [hidden]; y receives moe_result [hidden] (the
 * residual add stays with the caller); ids/probs receive the routes in
 * order [top_k].  Non-finite router logits return RUNTIME_ERROR, as
 * route_experts throws (:270-276).  Host buffers; synchronous. */
pk_hip_status pk_hip_moe_decode(pk_hip_ctx* ctx, const pk_hip_moe_layer* layer, const float* x,
                                float* y, uint32_t* ids, float* probs, char* error_buffer,
                                size_t error_capacity);

/* The host libm's expf results where they differ from the correctly
 * rounded exponential, as (input bits, result bits) pairs with increasing
 * inputs (the file libm_expf.bin the build writes beside the library: "PKEXPF01",
 * a uint32 count, then the pairs), for the context's reference-order kernels
 * (pk_hip_moe_decode_reference_order).  count 0 clears the table; without
 * one, those kernels' expf is the correctly rounded exponential. */
pk_hip_status pk_hip_set_libm_expf(pk_hip_ctx* ctx, const uint32_t* libm_expf_pairs,
                                   uint64_t pair_count, char* error_buffer,
                                   size_t error_capacity);

/* pk_hip_moe_decode in the reference's own operation order (the MoE block of
 * src/qwen3_moe_runner.cpp:644-691 with route_experts :267-305): the router
 * logits as linear's serial FP32 sums, route_experts' ranking and FP64
 * softmax, linear_k / linear_quantized's block-order sums for gate, up and
 * down, g / (1 + expf(-g)) * u with the host libm's expf (pk_hip_set_libm_expf),
 * and moe_result += p * expert_output in route order from zero -- bit for bit
 * the reference's outputs.  Qwen3-MoE layers (scale 1) up to 256 experts,
 * top-16 and rows of 8192; others return UNSUPPORTED.  Host buffers;
 * synchronous. */
pk_hip_status pk_hip_moe_decode_reference_order(pk_hip_ctx* ctx, const pk_hip_moe_layer* layer,
                                                const float* x, float* y, uint32_t* ids,
                                                float* probs, char* error_buffer,
                                                size_t error_capacity);

/* Device-buffer variant, enqueued on `stream` without synchronising.  A
 * router error is reported by the next pk_hip_sync.  Scratch and stream
 * capture as for pk_hip_moe_prefill_async. */
pk_hip_status pk_hip_moe_decode_async(pk_hip_ctx* ctx, const pk_hip_moe_layer* layer,
                                      const float* device_x, float* device_y,
                                      uint32_t* device_ids, float* device_probs, void* stream,
                                      char* error_buffer, size_t error_capacity);

/* pk_hip_moe_decode_async that also records its phase times (no
 * counterpart in the reference; a trace of the reference runner's MoE block
 * step for performance work): every wave's lane 0 reads the 100 MHz
 * s_memrealtime counter at fixed points of each kernel into `device_trace`,
 * PK_HIP_TRACE_WORDS uint64 words, word (kernel * 8192 + wave) * 8 + slot with
 * kernel 0 router (slots: start, inputs in, done), 1 gate/up (start, ranked,
 * routes shared, weight loads issued, done), 2 down (start, loads issued,
 * dots done, partials shared, done) and wave = workgroup * waves per
 * workgroup + wave.  Words of waves that do not exist keep their contents. */
#define PK_HIP_TRACE_WORDS (3u * 8192u * 8u)
pk_hip_status pk_hip_moe_decode_traced_async(pk_hip_ctx* ctx, const pk_hip_moe_layer* layer,
                                             const float* device_x, float* device_y,
                                             uint32_t* device_ids, float* device_probs,
                                             uint64_t* device_trace, void* stream,
                                             char* error_buffer, size_t error_capacity);

/* As pk_hip_moe_decode_async, allocating nothing: no counterpart in the
 * reference; for callers that cannot allocate device memory (code under HIP
 * graph capture, tight serving loops, harnesses that forbid hipMalloc).  The
 * router sums, activations and status words live in one static device array
 * of 69,888 bytes per GPU, so layers above 256 experts, top_k 8 or ffn 2048
 * are rejected with INVALID_ARGUMENT.  Every call on a GPU shares that array:
 * calls that overlap on one GPU (two streams, two contexts) race.  A
 * non-finite router logit is reported through the outputs (ids UINT32_MAX,
 * probs 0), not by pk_hip_sync. */
pk_hip_status pk_hip_moe_decode_noalloc(pk_hip_ctx* ctx, const pk_hip_moe_layer* layer,
                                        const float* device_x, float* device_y,
                                        uint32_t* device_ids, float* device_probs, void* stream,
                                        char* error_buffer, size_t error_capacity);

/* Qwen3.5-MoE block for one token (src/qwen35_runner.cpp:670-764) on the same
 * kernels.  Routed experts come from select_experts (:131-173): the same
 * top-k order as route_experts (ids bit-exact), weights from an FP32 softmax
 * over all experts, optional FP32 renormalisation (routed.normalize =
 * expert_weights_norm), then times routed.scale (expert_weights_scale).
 * Activations are silu(g) * u (:111-123).  The shared expert is added last
 * with weight sigmoid(shared_router . x).  shared_router is F32 [hidden]
 * (ffn_gate_inp_shexp, uploaded as [hidden, 1]); shared_gate/shared_up
 * [hidden, ffn] and shared_down [ffn, hidden] (ffn_*_shexp) must have the
 * routed experts' types and ffn width (top_k <= 8 as for
 * pk_hip_moe_decode), else UNSUPPORTED.  y
 * receives mixer_output (:759-761); ids/weights the routes in order (weights
 * include the scale).  Host buffers; synchronous. */
typedef struct pk_hip_moe35_layer {
    pk_hip_moe_layer routed;
    const pk_hip_weight* shared_router;
    const pk_hip_weight* shared_gate;
    const pk_hip_weight* shared_up;
    const pk_hip_weight* shared_down;
} pk_hip_moe35_layer;

pk_hip_status pk_hip_moe35_decode(pk_hip_ctx* ctx, const pk_hip_moe35_layer* layer,
                                  const float* x, float* y, uint32_t* ids, float* weights,
                                  char* error_buffer, size_t error_capacity);

/* Device-buffer variant, enqueued on `stream` without synchronising. */
pk_hip_status pk_hip_moe35_decode_async(pk_hip_ctx* ctx, const pk_hip_moe35_layer* layer,
                                        const float* device_x, float* device_y,
                                        uint32_t* device_ids, float* device_weights, void* stream,
                                        char* error_buffer, size_t error_capacity);

/* A batch of tokens through one MoE layer: the prompt loop of the reference
 * (src/qwen3_moe_runner.cpp:785-790), whose tokens each take the MoE block
 * (:644-691) independently.  x [tokens][hidden] holds the normalised hidden
 * states; y [tokens][hidden], ids and probs [tokens][top_k] receive each
 * token's moe_result and routes, equal to pk_hip_moe_decode's for that token
 * (ids bit-exact, outputs within FP32 reassociation).  Tokens are grouped per
 * expert; the expert products run on bf16 MFMA with exact products (FP32
 * activations split into three bf16 parts, the quantised weights as exact
 * bf16 integers, scales applied per group in FP32).  1 <= tokens <=
 * 4096; gate/up and down of any K-quant/Q8_0/Q4_0/Q4_1 type, ffn a multiple of
 * 256.  Host buffers; synchronous.  Non-finite router logits return
 * RUNTIME_ERROR. */
pk_hip_status pk_hip_moe_prefill(pk_hip_ctx* ctx, const pk_hip_moe_layer* layer, const float* x,
                                 uint32_t tokens, float* y, uint32_t* ids, float* probs,
                                 char* error_buffer, size_t error_capacity);

/* Device-buffer variant, enqueued on `stream` without synchronising.  The
 * first call for a given batch shape allocates the context's scratch; capture
 * it into a HIP graph only after one such call: a call under stream capture
 * that would need more scratch returns INVALID_ARGUMENT.  When a later call
 * needs more, the context allocates anew and keeps the old scratch until
 * pk_hip_destroy, so graphs captured earlier stay valid.  Every *_async call
 * on one context shares that scratch: enqueue them on one stream (or order
 * them yourself), as a replayed graph uses the scratch it captured. */
pk_hip_status pk_hip_moe_prefill_async(pk_hip_ctx* ctx, const pk_hip_moe_layer* layer,
                                       const float* device_x, uint32_t tokens, float* device_y,
                                       uint32_t* device_ids, float* device_probs, void* stream,
                                       char* error_buffer, size_t error_capacity);

/* The Qwen3.5-MoE block (pk_hip_moe35_decode) for a batch of tokens: the
 * reference runner's prompt loop takes the block once per token
 * (src/qwen35_runner.cpp:670-764 per position).  The shared expert is one
 * more expert group that every token joins; its output is added after the
 * routed sum with weight sigmoid(shared_router . x).  ids/weights are
 * [tokens][top_k] (routed experts).  Same limits as pk_hip_moe_prefill and
 * pk_hip_moe35_decode; synchronous, host buffers. */
pk_hip_status pk_hip_moe35_prefill(pk_hip_ctx* ctx, const pk_hip_moe35_layer* layer,
                                   const float* x, uint32_t tokens, float* y, uint32_t* ids,
                                   float* weights, char* error_buffer, size_t error_capacity);

/* Device-buffer variant, enqueued on `stream` without synchronising. */
pk_hip_status pk_hip_moe35_prefill_async(pk_hip_ctx* ctx, const pk_hip_moe35_layer* layer,
                                         const float* device_x, uint32_t tokens, float* device_y,
                                         uint32_t* device_ids, float* device_weights, void* stream,
                                         char* error_buffer, size_t error_capacity);

/* ---- Whole-model greedy decode (Qwen3-MoE) ------------------------------------
 * Qwen3MoeRunner (include/pokitlms/model/qwen3_moe_runner.hpp:57-110) with
 * every layer of a token step on the GPU: forward_into
 * (src/qwen3_moe_runner.cpp:580-704) per token, greedy first-max argmax
 * (sample_token at temperature 0, :320-333), FP16 KV ring of kv_capacity
 * positions (the runner's context window, :372-376; kv_cache.cpp:131-294).
 * All weights are pk_hip_weight handles already resident on the context's
 * device; norm vectors are F32 [n, 1] uploads. */
typedef struct pk_hip_qwen3moe pk_hip_qwen3moe;

typedef struct pk_hip_qwen3moe_config {
    uint32_t layers, hidden, heads, kv_heads, head_dim; /* qwen3moe.* GGUF keys */
    uint32_t experts, top_k, ffn, vocab;
    uint32_t kv_capacity;                               /* <= 8192 positions */
    uint32_t context;                                   /* qwen3moe.context_length */
    uint32_t normalize;                                 /* expert_weights_norm */
    /* Non-zero: every kernel repeats the CPU's operation order (serial FP32
     * sums as linear_k/rms_norm/KvCache::attend, route_experts over serial
     * logits, RoPE table from the host libm), so greedy tokens track the
     * reference through router and logit near-ties.  Zero: the bandwidth-
     * optimised kernels (outputs within FP32 reassociation error). */
    uint32_t reference_order;
    float rms_eps, rope_theta;
    /* reference_order only: the host libm's expf results that differ from the
     * correctly rounded exponential, as (input bits, result bits) pairs in
     * increasing input-bit order (pokitlms_amd/host/expf_table.c writes them;
     * glibc: 170,648 pairs).  The softmax and SwiGLU exponentials then return
     * the CPU's bits (kv_cache.cpp:249, qwen3_moe_runner.cpp:683).  Count 0:
     * the correctly rounded value everywhere. */
    const uint32_t* libm_expf_pairs;
    uint64_t libm_expf_count;
} pk_hip_qwen3moe_config;

typedef struct pk_hip_qwen3moe_layer {
    const pk_hip_weight *attn_norm, *q, *q_norm, *k, *k_norm, *v, *o, *ffn_norm;
    const pk_hip_weight *router, *gate, *up, *down; /* as pk_hip_moe_layer */
} pk_hip_qwen3moe_layer;

typedef struct pk_hip_qwen3moe_weights {
    const pk_hip_weight *token_embd, *output_norm, *output;
    const pk_hip_qwen3moe_layer* layers; /* [config.layers] */
} pk_hip_qwen3moe_weights;

typedef struct pk_hip_generation_stats {
    uint64_t prefill_ns;      /* host wall time of the prompt forwards */
    uint64_t decode_ns;       /* device time of the decode forwards (HIP events) */
    uint32_t prompt_tokens;
    uint32_t decode_forwards; /* n_new - 1: the first token comes from the prompt's logits */
} pk_hip_generation_stats;

/* Validates shapes against the reference index (src/qwen3_moe_index.cpp:37-85)
 * and builds the device state; the weights must outlive the model. */
pk_hip_status pk_hip_qwen3moe_create(pk_hip_ctx* ctx, const pk_hip_qwen3moe_config* config,
                                     const pk_hip_qwen3moe_weights* weights,
                                     pk_hip_qwen3moe** out_model, char* error_buffer,
                                     size_t error_capacity);
void pk_hip_qwen3moe_destroy(pk_hip_qwen3moe* model);

/* generate_tokens (qwen3_moe_runner.hpp:74-78) at temperature 0 without an EOS
 * stop: resets the state, feeds the prompt at positions 0.., then writes n_new
 * greedy tokens to out_tokens.  last_logits (optional, vocab floats) receives
 * the logits after the last prompt token.  Non-finite router logits or
 * logits return RUNTIME_ERROR (route_experts and sample_token throw). */
pk_hip_status pk_hip_qwen3moe_generate(pk_hip_qwen3moe* model, const uint32_t* prompt,
                                       uint32_t n_prompt, uint32_t n_new, uint32_t* out_tokens,
                                       float* last_logits, pk_hip_generation_stats* stats,
                                       char* error_buffer, size_t error_capacity);

/* Seeded synthetic weights made in HBM (no counterpart in the reference: the
 * benchmark and test models, byte-identical to pokitlms_amd/synth_model.py):
 * word i = splitmix64(key + i), then the scale fix-up `kind` (0 none, 1
 * K-quant, 2 Q6_K, 3 F32 norm, 4 F32 router). */
pk_hip_status pk_hip_synth_weight(pk_hip_ctx* ctx, uint32_t ggml_type, uint64_t in, uint64_t out,
                                  uint32_t n_experts, uint64_t key, uint32_t kind,
                                  pk_hip_weight** out_weight, char* error_buffer,
                                  size_t error_capacity);

/* Rows [first_row, first_row + rows) of a resident weight as FP32 into host
 * memory (rows * in floats; expert selects a slice of an expert tensor,
 * UINT32_MAX for a plain matrix): TensorReader::read_float_rows_into for
 * F32/F16/BF16 (src/tensor_reader.cpp:164-198) and dequantize_quantized_row
 * for the quantized types (src/quantized_linear.cpp:427-493), bit for bit; the
 * device decode the embedding row and the kernels' scales use. */
pk_hip_status pk_hip_dequantize_rows(pk_hip_ctx* ctx, const pk_hip_weight* weight,
                                     uint32_t expert, uint64_t first_row, uint32_t rows,
                                     float* out, char* error_buffer, size_t error_capacity);

/* out[r] = rms_norm(x[r], w, eps) for rows r < rows of n values
 * (src/rms_norm.cpp:9-27): the serial FP32 sum of the squares x_i * x_i,
 * scale = 1 / sqrt(sum / n + eps), out_i = (x_i * scale) * w_i -- bit for bit
 * the reference's result, with the same kernel the reference-order decode
 * uses for its norms.  Host buffers x and out [rows][n], w [n]; n <= 8192. */
pk_hip_status pk_hip_rmsnorm(pk_hip_ctx* ctx, const float* x, const float* w, uint32_t rows,
                             uint32_t n, float eps, float* out, char* error_buffer,
                             size_t error_capacity);

/* Checksums of the reference-order decode's expf (no counterpart in the
 * reference; it pins the device side of the host libm's expf, which the
 * reference calls in the softmax and SwiGLU, src/kv_cache.cpp:249,
 * src/qwen3_moe_runner.cpp:683): the exponential in double rounded once to
 * float, replaced from the (input bits, result bits) pairs as
 * pk_hip_qwen3moe_config.libm_expf_pairs.  Block k covers the float bit
 * patterns b = first_bits + k * block_size + i, i < block_size, and sums[k] =
 * sum over i of (((uint64) result_bits << 32) | b) * 0xD6E8FEB86659FD93 mod
 * 2^64, so a host evaluating its libm the same way compares n_blocks words. */
pk_hip_status pk_hip_expf_block_sums(pk_hip_ctx* ctx, const uint32_t* libm_expf_pairs,
                                     uint64_t pair_count, uint32_t first_bits,
                                     uint32_t block_size, uint32_t n_blocks, uint64_t* sums,
                                     char* error_buffer, size_t error_capacity);

/* The fast decode step's residual add + RMSNorm kernel (no counterpart
 * name in the reference; it computes the runner's `hidden += delta`
 * followed by rms_norm(hidden, w), src/qwen3_moe_runner.cpp:630,692 and
 * src/rms_norm.cpp:9-27, for each of `rows` rows of n values): hidden_out =
 * hidden + delta (delta may be NULL), bit for bit; out = (hidden_out *
 * scale) * w with scale = 1 / sqrt(sum / n + eps), the sum of squares
 * reassociated as a block reduction (within FP32 reassociation error of the
 * reference's serial sum).  Host buffers [rows][n], w [n]. */
pk_hip_status pk_hip_add_rmsnorm(pk_hip_ctx* ctx, const float* hidden, const float* delta,
                                 const float* w, uint32_t rows, uint32_t n, float eps,
                                 float* hidden_out, float* out, char* error_buffer,
                                 size_t error_capacity);

/* The fast decode step's q/k/v projection with the attention norm in its
 * staging (no counterpart name in the reference; it computes the runner's
 * `hidden += delta`, rms_norm(hidden, norm_w) and the projection that reads
 * it, src/qwen3_moe_runner.cpp:614-620,692 and src/rms_norm.cpp:9-27, in one
 * launch): hidden_out = hidden + delta (delta may be NULL), bit for bit; y =
 * W . ((hidden_out * scale) * norm_w) with the sum of squares reassociated
 * as in pk_hip_add_rmsnorm.  Host buffers of the weight's width (hidden,
 * delta, norm_w, hidden_out) and height (y); a plain matrix.  Returns
 * PK_HIP_STATUS_UNSUPPORTED where the one-launch kernel does not cover the
 * type or width (widths up to 4096, a multiple of 4). */
pk_hip_status pk_hip_matvec_add_rmsnorm(pk_hip_ctx* ctx, const pk_hip_weight* weight,
                                        const float* hidden, const float* delta,
                                        const float* norm_w, float eps, float* hidden_out,
                                        float* y, char* error_buffer, size_t error_capacity);

/* Attention of one layer as the whole-model decode computes it. */
typedef struct pk_hip_attention_config {
    uint32_t heads, kv_heads, head_dim;  /* head_dim 64, 128 or 256 */
    uint32_t capacity;                   /* KV ring positions */
    float rms_eps, rope_theta;
    /* 0: the fast mode's kernel (device expf); non-zero: reference order,
     * which needs the host libm's expf exceptions (as pk_hip_qwen3moe_config) */
    uint32_t reference_order;
    const uint32_t* libm_expf_pairs;
    uint64_t libm_expf_count;
} pk_hip_attention_config;

/* For positions t = 0 .. steps - 1 in turn, the decode's attention stage of
 * one layer (src/qwen3_moe_runner.cpp:610-628): rms_norm of every q and k head
 * (q_norm / k_norm [head_dim]), NeoX RoPE with prepare_qwen_rope's angles
 * (:141-155), the FP16 KvCache::append of k and v and KvCache::attend over
 * the last `capacity` positions (src/kv_cache.cpp:131-294).  q / out
 * [steps][heads * head_dim], k / v [steps][kv_heads * head_dim] host buffers
 * (the projections before the head norms). */
pk_hip_status pk_hip_attention_steps(pk_hip_ctx* ctx, const pk_hip_attention_config* config,
                                     const float* q_norm, const float* k_norm, uint32_t steps,
                                     const float* q, const float* k, const float* v, float* out,
                                     char* error_buffer, size_t error_capacity);

/* A plain streaming read of `bytes` device bytes at `src` on `stream`
 * (no counterpart in the reference: the measured floor of any kernel that
 * reads that many bytes from HBM, for the benchmark).  16-byte-aligned src,
 * bytes a multiple of 16; sink: one device word, written only for one
 * particular XOR of the data. */
pk_hip_status pk_hip_read_floor_async(pk_hip_ctx* ctx, const void* src, uint64_t bytes,
                                      uint32_t* sink, void* stream, char* error_buffer,
                                      size_t error_capacity);

/* Waits for the context's work (and `stream`, if not NULL) and reports any
 * deferred router error. */
pk_hip_status pk_hip_sync(pk_hip_ctx* ctx, void* stream, char* error_buffer,
                          size_t error_capacity);

pk_hip_status pk_hip_get_stats(const pk_hip_ctx* ctx, pk_hip_stats* out_stats);
void pk_hip_reset_stats(pk_hip_ctx* ctx);

/* Switches per-launch HIP-event timing (pk_hip_options.time_kernels) on or
 * off for later calls.  While on, every call synchronises its stream. */
pk_hip_status pk_hip_set_kernel_timing(pk_hip_ctx* ctx, int enabled);

#ifdef __cplusplus
}
#endif

#endif /* POKIT_HIP_H */
