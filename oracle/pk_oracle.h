/*
 * pk_oracle.h -- CPU restatement of the PokitLMs routed-MoE K-quant path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the parity checker for the HIP
 * backend: only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline
 * leg may load it.  The product path (pokitlms_amd) never links or calls it.
 *
 * Every function restates the reference's x86-64 CPU arithmetic order
 * (reference built with -O3 and no -march, so no FMA contraction and the
 * scalar branches of src/simd_kernels.hpp).  Citations are to the reference
 * checkout (RemydreScarlet/PokitLMs v0.4.0).
 *
 * Return codes follow pokitlms_status (include/pokitlms/pokitlms.h:18-24):
 * 0 ok, 1 invalid argument, 2 runtime error.
 */
#ifndef PK_ORACLE_H
#define PK_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* GGUF tensor type ids (reference src/gguf_reader.cpp:21-57). */
enum {
    PKO_F32 = 0, PKO_F16 = 1, PKO_Q4_0 = 2, PKO_Q4_1 = 3, PKO_Q5_0 = 6, PKO_Q5_1 = 7,
    PKO_Q8_0 = 8, PKO_Q2_K = 10, PKO_Q3_K = 11, PKO_Q4_K = 12, PKO_Q5_K = 13, PKO_Q6_K = 14,
    PKO_BF16 = 30
};

/* Elements and bytes of one encoded block; 0 when the type is not on the path. */
uint32_t pko_block_elements(uint32_t type);
uint32_t pko_block_bytes(uint32_t type);

/* IEEE binary16 -> binary32, subnormals/Inf/NaN included
 * (src/quantized_linear.cpp:18-39). */
float pko_half_to_float(uint16_t bits);

/* One 256-element K-quant block to F32 (src/quantized_linear.cpp:166-205,
 * 286-328, 330-358). */
void pko_decode_q4_k(const uint8_t* block, float* out256);
void pko_decode_q5_k(const uint8_t* block, float* out256);
void pko_decode_q6_k(const uint8_t* block, float* out256);

/* One 32-element Q4_1 block to F32: fl(fl(q * d) + m), low nibbles first
 * (decode_q4_1, src/quantized_linear.cpp:53-62). */
void pko_decode_q4_1(const uint8_t* block, float* out32);

/* One 32-element Q5_0 / Q5_1 block (decode_q5_0 / decode_q5_1,
 * src/quantized_linear.cpp:64-77, 79-93) and one 256-element Q2_K / Q3_K
 * block (decode_q2_k / decode_q3_k, :95-121, 123-164) to F32. */
void pko_decode_q5_0(const uint8_t* block, float* out32);
void pko_decode_q5_1(const uint8_t* block, float* out32);
void pko_decode_q2_k(const uint8_t* block, float* out256);
void pko_decode_q3_k(const uint8_t* block, float* out256);

/* dequantize_quantized_row for every quantized type above
 * (src/quantized_linear.cpp:427-493). */
int pko_dequantize_row(uint32_t type, const uint8_t* encoded, uint64_t encoded_bytes,
                       float* out, uint64_t count);

/* out[r] = W[r] . x for a row-major GGUF matrix [in, rows] of the given type:
 * the tensor_linear CPU branch (src/tensor_linear.cpp:232-263) over
 * linear_k / linear_quantized / linear (src/quantized_linear.cpp:360-423,
 * src/linear.cpp:10-31).  Single-threaded; rows are independent, so the
 * reference's row thread pool does not change any bit. */
int pko_linear(uint32_t type, const uint8_t* weights, uint64_t weight_bytes,
               uint64_t in, uint64_t rows, const float* x, float* y);

/* route_experts (src/qwen3_moe_runner.cpp:267-305): double softmax
 * denominator over all logits, top-k ordered by (logit desc, id asc),
 * float probabilities, optional float renormalisation.  Returns 2 on
 * non-finite logits, 1 on a bad top_k. */
int pko_route_experts(const float* logits, uint32_t count, uint32_t top_k, int normalize,
                      uint32_t* ids, float* selected_logits, float* probabilities);

/* One Qwen3-MoE MoE block for a single token (src/qwen3_moe_runner.cpp:643-692):
 * router logits (F32 [hidden, n_experts]) -> route_experts -> for each route in
 * order: gate/up matvec, SwiGLU g/(1+expf(-g))*u, down matvec, moe += p*y.
 * Expert tensors are the GGUF [in, out, E] layout, expert e at byte e*slice.
 * y receives moe_result (the residual add is the caller's). */
int pko_moe_block(const float* router, uint32_t hidden, uint32_t n_experts, uint32_t ffn,
                  uint32_t gate_type, const uint8_t* gate, uint32_t up_type, const uint8_t* up,
                  uint32_t down_type, const uint8_t* down, uint32_t top_k, int normalize,
                  const float* x, float* y, uint32_t* ids, float* probabilities);

/* select_experts (src/qwen35_runner.cpp:131-173): FP32 softmax over all
 * logits (expf of logit - max, FP32 denominator summed in id order, FP32
 * division), top-k by (logit desc, id asc), weights the selected
 * probabilities, optional FP32 renormalisation.  Returns 2 on non-finite
 * logits or an invalid softmax / selected sum, 1 on a bad top_k. */
int pko_select_experts(const float* logits, uint32_t count, uint32_t top_k, int normalize,
                       uint32_t* ids, float* weights);

/* The Qwen3.5-MoE block for one token (src/qwen35_runner.cpp:690-761):
 * select_experts over the F32 router; per route in order gate/up,
 * silu(g) * u (sigmoid :111-115, silu :123), down, moe += (w * scale) * y;
 * then the shared expert: gate value = shared_router . x, gate/up [hidden,
 * shared_ffn], silu, down [shared_ffn, hidden], mixer = moe + sigmoid(gate
 * value) * y_shared.  y receives mixer_output; weights the route weights
 * before the scale. */
int pko_moe35_block(const float* router, uint32_t hidden, uint32_t n_experts, uint32_t ffn,
                    uint32_t gate_type, const uint8_t* gate, uint32_t up_type, const uint8_t* up,
                    uint32_t down_type, const uint8_t* down, uint32_t top_k, int normalize,
                    float scale, const float* shared_router, uint32_t shared_ffn,
                    uint32_t sgate_type, const uint8_t* sgate, uint32_t sup_type,
                    const uint8_t* sup, uint32_t sdown_type, const uint8_t* sdown,
                    const float* x, float* y, uint32_t* ids, float* weights);

/* rms_norm of each row (src/rms_norm.cpp:9-27): serial FP32 sum of squares,
 * scale = 1 / sqrt(sum / n + eps), out_i = (x_i * scale) * w_i. */
int pko_rms_norm(const float* x, const float* w, uint64_t rows, uint64_t n, float eps,
                 float* out);

/* The host libm's expf over float bit patterns, as block checksums: block k
 * covers b = first_bits + k * block_size + i (i < block_size) and sums[k] =
 * sum over i of (((uint64) bits(expf(x_b)) << 32) | b) * 0xD6E8FEB86659FD93
 * mod 2^64 (the device's pk_hip_expf_block_sums computes the same over its
 * expf).  The reference calls this libm's expf in the softmax and SwiGLU
 * (src/kv_cache.cpp:249, src/qwen3_moe_runner.cpp:683).  threads > 0 splits
 * the blocks over that many threads. */
void pko_expf_block_sums(uint32_t first_bits, uint32_t block_size, uint32_t n_blocks,
                         uint64_t* sums, uint32_t threads);


/* One layer's attention for positions 0 .. steps - 1 as the runner's token
 * step (src/qwen3_moe_runner.cpp:610-628): q/k head rms_norm, NeoX RoPE
 * (prepare_qwen_rope :141-155, rope_rotate_f32 src/simd_kernels.hpp:88-108),
 * FP16 KvCache::append and KvCache::attend (src/kv_cache.cpp:131-294) over a
 * ring of `capacity` positions.  q/out [steps][heads][head_dim], k/v
 * [steps][kv_heads][head_dim] (projections before the head norms). */
int pko_attention_steps(uint32_t heads, uint32_t kv_heads, uint32_t head_dim, uint32_t capacity,
                        float eps, float theta, const float* q_norm, const float* k_norm,
                        uint32_t steps, const float* q, const float* k, const float* v,
                        float* out);

/* hidden += delta (FP32, delta may be null), then out = rms_norm(hidden, w)
 * per row: the runner's residual add followed by its next RMSNorm
 * (src/qwen3_moe_runner.cpp:630,692; src/rms_norm.cpp:9-27). */
int pko_add_rms_norm(float* hidden, const float* delta, const float* w, uint64_t rows, uint64_t n,
                     float eps, float* out);

#ifdef __cplusplus
}
#endif

#endif
