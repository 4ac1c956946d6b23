// launch.hpp -- host-side entry points of the HIP kernels (no torch types).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace pk {

// Bytes each kernel may read past the end of a weight payload (2-byte-aligned
// formats fetch one extra dword); every device weight buffer is padded by it.
constexpr uint64_t kWeightTailPad = 64;

// Whether a kernel covers (type, in, batch): the register-resident kernels up
// to a width per batch size, the MFMA kernel for 5-8 vectors at any width it
// can split into at most 16 waves; wider rows are reported unsupported.
bool matvec_supported(uint32_t type, uint32_t in, uint32_t batch);

// y[b][r] = W[r] . x[b] for b < batch.  W: rows x row_bytes encoded GGUF rows
// (device), x: batch x in floats (device, rows 16-byte aligned), y: batch x rows.
// `partial`: device scratch of matvec_partial_floats(type, in, batch, rows)
// floats (K-sliced batched kernels; may be null where that count is 0).
hipError_t launch_matvec(uint32_t type, const uint8_t* W, uint64_t row_bytes, uint32_t rows,
                         uint32_t in, const float* x, float* y, uint32_t batch,
                         hipStream_t stream, float* partial = nullptr);
size_t matvec_partial_floats(uint32_t type, uint32_t in, uint32_t batch, uint32_t rows);

// One vector whose x is the RMSNorm of h + delta, computed by every workgroup
// of the matvec in its staging: x = (v * scale) * w with v = h + delta (delta
// null: v = h) and scale = 1 / sqrt(mean(v^2) + eps); v is written to h_out
// (device, may be null; not h or delta).  in a multiple of 4, at most 4096.
struct MatvecNorm {
    const float* delta;
    const float* w;
    float* h_out;
    float eps;
};
// hipErrorNotSupported (nothing launched) where the staged one-vector kernel
// does not cover (type, in): the caller norms and multiplies separately.
hipError_t launch_matvec_norm(uint32_t type, const uint8_t* W, uint32_t rows, uint32_t in,
                              const float* h, const MatvecNorm& nm, float* y,
                              hipStream_t stream);

// Batched matvecs on MFMA (matvec_mfma.hip): 256-value K ranges per wave for
// (type, in, batch), 0 where that kernel does not apply; launch_matvec takes
// it where matvec_mfma_takes says so.
uint32_t matvec_mfma_blocks_per_wave(uint32_t type, uint32_t in, uint32_t batch);
bool matvec_mfma_takes(uint32_t type, uint32_t in, uint32_t batch, uint32_t rows);
size_t matvec_mfma_partial_floats(uint32_t type, uint32_t in, uint32_t batch, uint32_t rows);
hipError_t launch_matvec_mfma(uint32_t type, const uint8_t* W, uint32_t rows, uint32_t in,
                              const float* x, float* y, uint32_t batch, hipStream_t stream,
                              float* partial);

// One single-token routed-MoE layer (router -> top-k -> gate/up SwiGLU ->
// down -> weighted combine).  Device pointers throughout.
struct MoeDecodeArgs {
    const float* router;    // F32 [n_experts][hidden]
    const uint8_t* gate;    // expert-major slices
    const uint8_t* up;
    const uint8_t* down;
    uint32_t gate_type, up_type, down_type;
    uint64_t gate_slice, up_slice, down_slice;     // bytes per expert
    uint64_t gate_row, up_row, down_row;           // bytes per row
    uint32_t hidden, ffn, n_experts, top_k;
    uint32_t normalize;
    float scale;
    // Qwen3.5-MoE (variant 1): select_experts weights, silu activations and
    // the shared expert as route top_k (the routed experts' types and rows),
    // weighted by sigmoid(shared_router . x) (router row n_experts)
    uint32_t variant;
    const float* shared_router;   // F32 [hidden]
    const uint8_t* shared_gate;
    const uint8_t* shared_up;
    const uint8_t* shared_down;
    const float* x;          // [hidden]
    float* y;                // [hidden] moe_result
    uint32_t* ids;           // [top_k] route order
    float* probs;            // [top_k]
    // context scratch (device)
    double* row_sum;         // [n_experts + variant]
    double* row_bound;       // [n_experts + variant]
    float* act;              // [top_k + variant][ffn]
    uint32_t* status;        // [4]: error flag, serial-fallback count, candidates, spare
    // optional phase times (null: off): see kTraceWaves
    uint64_t* trace;
};

// Phase times of a traced decode step: the 100 MHz s_memrealtime counter
// read by lane 0 of every wave at fixed points, trace[(kernel * kTraceWaves
// + wave) * kTraceSlots + slot] with kernel 0 router, 1 gate/up, 2 down and
// wave = blockIdx.x * (waves per workgroup) + wave in the workgroup.
constexpr uint32_t kTraceWaves = 8192;
constexpr uint32_t kTraceSlots = 8;
constexpr uint64_t kTraceWords = 3ull * kTraceWaves * kTraceSlots;

bool moe_decode_supported(uint32_t gate_type, uint32_t up_type, uint32_t down_type,
                          uint32_t hidden, uint32_t ffn, uint32_t n_experts, uint32_t top_k,
                          uint32_t variant = 0);
hipError_t launch_moe_decode(const MoeDecodeArgs& a, hipStream_t stream);

// Batched prefill: tokens independent single-token MoE blocks, grouped per
// expert for MFMA GEMMs.  Scratch sizes for `tokens` tokens (T), top_k (K),
// n_experts (E), pairs P = T*K: row_sum/row_bound T*E, offsets E+1, tiles and
// n_tiles moe_prefill_max_tiles(T, K, E) + 1, perm P, x_parts 3*T*hidden,
// x_sums T*hidden/16, act_parts 3*P*ffn, act_sums P*ffn/16,
// out P*hidden.  Variant 1 (Qwen3.5) adds the shared expert as one more
// route per token and one more router row and expert group: K = top_k + 1 and
// E = n_experts + 1 in these sizes.
constexpr uint32_t kMaxPrefillTokens = 4096;
struct MoePrefillArgs {
    MoeDecodeArgs layer;     // weights, shapes, top_k, normalize, scale
    uint32_t tokens, max_tiles;
    const float* x;          // [tokens][hidden]
    float* y;                // [tokens][hidden]
    uint32_t* ids;           // [tokens][top_k]
    float* probs;            // [tokens][top_k]
    double* row_sum;         // [tokens][n_experts]
    double* row_bound;
    uint32_t* offsets;       // [n_experts + 1]
    uint32_t* tiles;         // [max_tiles]
    uint32_t* n_tiles;       // [1]
    uint32_t* perm;          // [P]: grouped row -> token * top_k + route
    uint16_t* x_parts;       // 3 bf16 planes [tokens][hidden]: x = hi + mid + lo
    float* x_sums;           // [tokens][hidden / G]: sums over gate/up scale groups
    uint16_t* act_parts;     // 3 bf16 planes [P][ffn], grouped rows (gate/up epilogue)
    float* act_sums;         // [P][ffn / G]: sums over down scale groups
    float* out;              // [P][hidden], slot token * top_k + route
    uint32_t* status;        // as MoeDecodeArgs::status
};
uint32_t moe_prefill_max_tiles(uint32_t tokens, uint32_t top_k, uint32_t n_experts);
bool moe_prefill_supported(uint32_t gate_type, uint32_t up_type, uint32_t down_type,
                           uint32_t hidden, uint32_t ffn, uint32_t n_experts, uint32_t top_k,
                           uint32_t tokens, uint32_t variant = 0);
// The prefill's launches in three phases (timed separately): routing and
// grouping (router, ranking, grouping), the gate/up GEMMs, and down + combine.
hipError_t launch_prefill_routing(const MoePrefillArgs& a, hipStream_t stream);
hipError_t launch_prefill_gate_up(const MoePrefillArgs& a, hipStream_t stream);
hipError_t launch_prefill_down(const MoePrefillArgs& a, hipStream_t stream);

// Whole-model greedy decode (Qwen3-MoE).  One step = one token through every
// layer; the step's position and token are read from `state` and `tokens` in
// device memory, so a captured step graph replays for every token.
constexpr uint32_t kMaxModelContext = 8192;  // KV ring positions (attention scores in LDS)
struct ModelLayer {
    const float* attn_norm;   // [hidden]
    const float* q_norm;      // [head_dim]
    const float* k_norm;
    const float* ffn_norm;    // [hidden]
    const uint8_t* q;         // [heads * head_dim] rows of [hidden]
    const uint8_t* k;         // [kv_heads * head_dim] rows
    const uint8_t* v;
    const uint8_t* qkv;       // fast mode: q, k and v rows back to back, or null
    const uint8_t* o;         // [hidden] rows of [heads * head_dim]
    uint32_t attn_type;
    uint64_t q_row, k_row, v_row, o_row;
    uint16_t* kcache;         // FP16 [capacity][kv_heads][head_dim]
    uint16_t* vcache;
    MoeDecodeArgs moe;        // x = the normed state, y = this layer's MoE output
};
// The host libm's expf results that differ from the correctly rounded value,
// as a two-choice cuckoo table: input bits b sit at slots[h0(b)] of the first
// half or slots[h1(b)] of the second, h_t(b) = (b * mul_t) >> (32 - bits);
// a slot is (input bits, result bits), empty slots hold input 0xffffffff.
struct LibmExpf {
    const uint32_t* slots;    // [2][1 << bits][2], or null (no exceptions)
    uint32_t bits, mul0, mul1;
};
constexpr uint32_t kExpfEmpty = 0xffffffffu;

struct ModelArgs {
    uint32_t layers, hidden, heads, kv_heads, head_dim, vocab, capacity;
    uint32_t embd_type, out_type;
    uint64_t embd_row, out_row;
    float rms_eps, rope_theta, attn_scale;
    const uint8_t* embd;      // token_embd rows [vocab] of [hidden]
    const float* out_norm;
    const uint8_t* out;       // output head rows [vocab]
    uint32_t* state;          // [0] position, [1] prompt length, [2] non-finite logits flag
    uint32_t* tokens;         // prompt, then generated ids
    float* hidden_state;      // residual stream [hidden]
    float* normed;            // [hidden]
    float* q;                 // [heads * head_dim]
    float* k;                 // [kv_heads * head_dim]
    float* v;
    float* att;               // attention output [heads * head_dim]
    float* attn_out;          // [hidden]
    float* hidden_alt;        // reference order: the residual stream's second buffer
    float* logits;            // [vocab]
    float* argmax_part;       // per 2048-logit chunk: maximum, index bits
    // reference-order mode: every kernel repeats the CPU's operation order
    uint32_t exact;
    const float* rope_table;  // [positions][head_dim]: cos, then sin (host libm; both modes)
    float* ref_scratch;       // router logits, gate, up, expert outputs
    LibmExpf expf;            // reference order: the host libm's expf exceptions
};
bool model_supported(const ModelArgs& a);
// The fast step's residual add + RMSNorm (one workgroup): v = x + d (d may be
// null) into xo (null: x itself), out = (v * (1 / sqrt(sum(v^2) / n + eps))) * w
// with the sum of squares reassociated (a block reduction).
hipError_t launch_fast_add_rmsnorm(float* x, const float* d, const float* w, float* out, uint32_t n,
                                   float eps, hipStream_t stream, float* xo = nullptr);
// logits: run the final norm, head and argmax (else only advance the position).
hipError_t launch_model_step(const ModelArgs& a, const ModelLayer* layers, bool logits,
                             hipStream_t stream);

// Rows [first_row, first_row + rows) of a slice (rows_in_slice rows of `in`
// elements) as FP32, decoded exactly as the embedding row (every type the
// embedding takes): out is rows * in floats (device).
bool dequant_rows_supported(uint32_t type, uint32_t in);
hipError_t launch_dequant_rows(uint32_t type, const uint8_t* slice, uint64_t rows_in_slice,
                               uint32_t in, uint64_t first_row, uint32_t rows, float* out,
                               hipStream_t stream);

// Checksums of the reference-order expf over float bit patterns: block k
// covers patterns first_bits + k * block_size + i (i < block_size) and sums
// (uint64) ((result bits << 32) | input bits) * 0xD6E8FEB86659FD93 mod 2^64.
hipError_t launch_expf_block_sums(const LibmExpf& t, uint32_t first_bits, uint32_t block_size,
                                  uint32_t n_blocks, unsigned long long* sums, hipStream_t stream);

// Seeded synthetic weight bytes (see pokitlms_amd/synth_model.py): kind 0 raw,
// 1 K-quant scale fix-up (block_bytes 144/176), 2 Q6_K, 3 F32 norm, 4 F32 router.
hipError_t launch_synth_fill(uint8_t* dst, uint64_t nbytes, uint64_t key, uint32_t kind,
                             uint32_t block_bytes, hipStream_t stream);

// Reference-order matvec: y[route][row] = row . x[route] summed as the CPU
// does (see exact.hip).  ids (optional) selects each route's expert slice.
constexpr uint32_t kMaxRefWidth = 8192;
constexpr uint32_t kMaxRefTopK = 16;
constexpr uint32_t kMaxExperts256 = 256;
// What an RMSNorm adds to the residual stream first: delta, or the
// route-order combine of the MoE block's expert outputs.
struct RefResidual {
    const float* delta;       // [n], or null
    const float* parts;       // [K][n] expert outputs, combined with probs in route order
    const float* probs;
    uint32_t K;
};
// An RMSNorm computed in a matvec's staging: every workgroup normalises
// x + residual into its LDS; the leader workgroup (0, 0) also writes the
// updated residual stream and/or the normed vector.
struct RefNormIn {
    const float* x;
    RefResidual res;
    const float* w;           // norm weights; null: no norm
    float* x_out;
    float* normed_out;
    float eps;
};
// route_experts in a matvec's prologue: every workgroup ranks the logits for
// its own route (blockIdx.y); the leader writes ids, probs and the status.
struct RefRouteIn {
    const float* logits;      // null: no routing (ids, if set, select the slices)
    uint32_t n_experts, top_k, normalize;
    uint32_t* ids;
    float* probs;
    uint32_t* status;
};

// Up to kMaxRefSegs matrices of one type and width in one launch: segment k
// covers workgroups [seg[k].block0, seg[k + 1].block0) along x.
constexpr uint32_t kMaxRefSegs = 3;
struct RefSeg {
    const uint8_t* W;
    uint64_t row_bytes, slice_bytes;
    uint32_t rows, block0;
    float* y;
};
struct RefMatvecArgs {
    const uint8_t* W;
    uint64_t row_bytes, slice_bytes;
    const uint32_t* ids;
    uint32_t rows, in;
    const float* x;
    uint64_t x_stride;
    float* y;
    uint64_t y_stride;
    // optional, set by launch_ref_matvec_multi / the SwiGLU staging
    uint32_t nseg;            // 0: the single matrix above
    RefSeg seg[kMaxRefSegs];
    const float* x_up;        // non-null: stage g / (1 + expf(-g)) * u, g = x, u = x_up
    float* act;               // non-null (with seg[0] gate, seg[1] up): write the SwiGLU activations
    LibmExpf expf;
    RefNormIn norm;           // norm.w set: x is RMSNorm(norm.x + norm.res) * norm.w
    RefRouteIn route;         // route.logits set: the expert slices come from routing
};
bool ref_matvec_supported(uint32_t type, uint32_t in);
hipError_t launch_ref_matvec(uint32_t type, const RefMatvecArgs& a, uint32_t routes,
                             hipStream_t stream);
// Several matrices sharing x (q/k/v; gate/up per route): one launch.
hipError_t launch_ref_matvec_multi(uint32_t type, RefMatvecArgs a, const RefSeg* segs, uint32_t n,
                                   uint32_t routes, hipStream_t stream);
// Gate and up of every route in one launch, each workgroup computing the same
// rows of both, with the SwiGLU activations g / (1 + expf(-g)) * u written to
// a.act (row stride a.y_stride) instead of the two outputs; false when the
// row is too wide for the pairing (then the caller launches the two
// matrices and stages the SwiGLU in the down projection).
bool ref_gate_up_act_supported(uint32_t type, uint32_t in);
hipError_t launch_ref_gate_up_act(uint32_t type, RefMatvecArgs a, const RefSeg& gate,
                                  const RefSeg& up, uint32_t routes, hipStream_t s);
hipError_t launch_ref_rmsnorm(float* x, const RefResidual& res, const float* w, float* out,
                              uint32_t n, uint32_t rows, float eps, hipStream_t stream);
// Head dims 64/128/256 and a KV window whose scores fit LDS beside a V tile.
bool ref_attention_supported(uint32_t head_dim, uint32_t capacity);
// Widths whose RMSNorm the matvec staging can carry.
constexpr uint32_t kMaxRefNormWidth = 4096;
// q/k head norms, RoPE, KV append and attention of one layer in the
// reference's order (both modes use it).
hipError_t launch_ref_attention(const ModelArgs& a, const ModelLayer& L, hipStream_t stream);
// The same attention with the device's expf (the fast step).
hipError_t launch_fast_attention(const ModelArgs& a, const ModelLayer& L, hipStream_t stream);
// The reference-order token step after the embedding (all layers, then the
// head when logits).
hipError_t launch_ref_step(const ModelArgs& a, const ModelLayer* layers, bool logits,
                           hipStream_t stream);
// The MoE block of one token in the reference's operation order (router rows,
// route_experts, gate/up, SwiGLU with the given expf, down, route-order
// combine; variant 0 only): m.x normalised input, m.y moe_result, m.ids /
// m.probs the routes, m.status the non-finite flag; scratch holds
// ref_scratch_floats(top_k, ffn, hidden) floats.
bool ref_moe_block_supported(const MoeDecodeArgs& m);
hipError_t launch_ref_moe_block(const MoeDecodeArgs& m, float* scratch, const LibmExpf& expf,
                                hipStream_t stream);
// floats of ModelArgs::ref_scratch for one layer shape
inline uint64_t ref_scratch_floats(uint32_t top_k, uint32_t ffn, uint32_t hidden) {
    return kMaxExperts256 + 2ull * top_k * ffn + static_cast<uint64_t>(top_k) * hidden;
}

// A plain streaming read of `bytes` bytes (16-byte nontemporal loads spread
// over the whole chip), the floor any kernel reading that many bytes from HBM
// meets: the XOR of the data goes to *sink only if it equals a constant
// (so no load can be dropped), 16-byte aligned src, bytes % 16 == 0.
hipError_t launch_read_floor(const uint8_t* src, uint64_t bytes, uint32_t* sink, hipStream_t stream);

// Individual stages (timing and tests).
hipError_t launch_moe_router(const MoeDecodeArgs& a, hipStream_t stream);
hipError_t launch_moe_gate_up(const MoeDecodeArgs& a, hipStream_t stream);
hipError_t launch_moe_down(const MoeDecodeArgs& a, hipStream_t stream);

}  // namespace pk
