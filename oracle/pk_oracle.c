/*
 * pk_oracle.c -- CPU restatement of the PokitLMs routed-MoE K-quant path.
 *
 * TEST INFRASTRUCTURE ONLY (parity checker and CPU-baseline port); the HIP
 * product path never calls it.  Build: oracle/Makefile (gcc -O3, no -march,
 * -ffp-contract=off), i.e. the same no-FMA scalar arithmetic as the reference
 * x86-64 build.  Each function names the reference lines it restates.
 *
 * Pinned by: tests/test_oracle.py (golden vectors written by the compiled
 * reference, tests/golden/make_golden.py; exhaustive binary16 check against
 * numpy; known-answer Q5_K blocks of tests/regression_test.cpp:86-112;
 * dyadic-exact closed forms for every decoder; brute-force routing order).
 */
#include "pk_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <pthread.h>
#include <string.h>

uint32_t pko_block_elements(uint32_t type) {
    switch (type) {
        case PKO_F32: case PKO_F16: case PKO_BF16: return 1;
        case PKO_Q4_0: case PKO_Q4_1: case PKO_Q5_0: case PKO_Q5_1: case PKO_Q8_0: return 32;
        case PKO_Q2_K: case PKO_Q3_K: case PKO_Q4_K: case PKO_Q5_K: case PKO_Q6_K: return 256;
        default: return 0;
    }
}

uint32_t pko_block_bytes(uint32_t type) {
    switch (type) {
        case PKO_F32: return 4;
        case PKO_F16: case PKO_BF16: return 2;
        case PKO_Q4_0: return 18;
        case PKO_Q4_1: return 20;
        case PKO_Q5_0: return 22;
        case PKO_Q5_1: return 24;
        case PKO_Q8_0: return 34;
        case PKO_Q2_K: return 84;
        case PKO_Q3_K: return 110;
        case PKO_Q4_K: return 144;
        case PKO_Q5_K: return 176;
        case PKO_Q6_K: return 210;
        default: return 0;
    }
}

static uint16_t rd16(const uint8_t* p) { return (uint16_t)(p[0] | (p[1] << 8)); }

static float bits_to_float(uint32_t u) {
    float f;
    memcpy(&f, &u, sizeof f);
    return f;
}

/* src/quantized_linear.cpp:18-39 */
float pko_half_to_float(uint16_t bits) {
    const uint32_t sign = (uint32_t)(bits & 0x8000u) << 16;
    const uint32_t exponent = (bits >> 10) & 0x1fu;
    uint32_t mantissa = bits & 0x03ffu;
    if (exponent == 0) {
        if (mantissa == 0) return bits_to_float(sign);
        int e = -14;
        while ((mantissa & 0x0400u) == 0) {
            mantissa <<= 1;
            --e;
        }
        mantissa &= 0x03ffu;
        return bits_to_float(sign | ((uint32_t)(e + 127) << 23) | (mantissa << 13));
    }
    if (exponent == 0x1fu) return bits_to_float(sign | 0x7f800000u | (mantissa << 13));
    return bits_to_float(sign | ((exponent + 112u) << 23) | (mantissa << 13));
}

/* 6-bit (scale, min) pair j of a Q4_K/Q5_K block, from the 12 packed bytes
 * (the scale_min lambda, src/quantized_linear.cpp:176-188). */
static void kq_scale_min(const uint8_t* sc, unsigned j, unsigned* s, unsigned* m) {
    if (j < 4) {
        *s = sc[j] & 63u;
        *m = sc[j + 4] & 63u;
    } else {
        *s = (sc[j + 4] & 0x0fu) | ((sc[j - 4] >> 6) << 4);
        *m = (sc[j + 4] >> 4) | ((sc[j] >> 6) << 4);
    }
}

/* src/quantized_linear.cpp:166-205: value = fl(fl(d*sc)*q) - fl(dmin*m). */
void pko_decode_q4_k(const uint8_t* block, float* out) {
    const float d = pko_half_to_float(rd16(block));
    const float dmin = pko_half_to_float(rd16(block + 2));
    const uint8_t* sc = block + 4;
    const uint8_t* qs = block + 16;
    unsigned o = 0;
    for (unsigned chunk = 0; chunk < 4; ++chunk) {
        unsigned s0, m0, s1, m1;
        kq_scale_min(sc, 2 * chunk, &s0, &m0);
        kq_scale_min(sc, 2 * chunk + 1, &s1, &m1);
        const float ds0 = d * (float)s0, dm0 = dmin * (float)m0;
        const float ds1 = d * (float)s1, dm1 = dmin * (float)m1;
        for (unsigned i = 0; i < 32; ++i) out[o++] = ds0 * (float)(qs[i] & 0x0fu) - dm0;
        for (unsigned i = 0; i < 32; ++i) out[o++] = ds1 * (float)(qs[i] >> 4) - dm1;
        qs += 32;
    }
}

/* src/quantized_linear.cpp:286-328: as Q4_K with a fifth bit from qh[32]. */
void pko_decode_q5_k(const uint8_t* block, float* out) {
    const float d = pko_half_to_float(rd16(block));
    const float dmin = pko_half_to_float(rd16(block + 2));
    const uint8_t* sc = block + 4;
    const uint8_t* qh = block + 16;
    const uint8_t* qs = block + 48;
    unsigned o = 0;
    unsigned mask1 = 1, mask2 = 2;
    for (unsigned chunk = 0; chunk < 4; ++chunk) {
        unsigned s0, m0, s1, m1;
        kq_scale_min(sc, 2 * chunk, &s0, &m0);
        kq_scale_min(sc, 2 * chunk + 1, &s1, &m1);
        const float ds0 = d * (float)s0, dm0 = dmin * (float)m0;
        const float ds1 = d * (float)s1, dm1 = dmin * (float)m1;
        for (unsigned i = 0; i < 32; ++i)
            out[o++] = ds0 * (float)((qs[i] & 0x0fu) + ((qh[i] & mask1) ? 16u : 0u)) - dm0;
        for (unsigned i = 0; i < 32; ++i)
            out[o++] = ds1 * (float)((qs[i] >> 4) + ((qh[i] & mask2) ? 16u : 0u)) - dm1;
        qs += 32;
        mask1 = (mask1 << 2) & 0xffu;
        mask2 = (mask2 << 2) & 0xffu;
        /* mask1 never reaches zero inside four chunks (the reference's
         * wrap at :326 is dead for one block), so qh is not advanced. */
    }
}

/* src/quantized_linear.cpp:330-358: value = fl(fl(d*s)*q), s int8, q in [-32,31]. */
void pko_decode_q6_k(const uint8_t* block, float* out) {
    const uint8_t* ql = block;
    const uint8_t* qh = block + 128;
    const int8_t* sc = (const int8_t*)(block + 192);
    const float d = pko_half_to_float(rd16(block + 208));
    for (unsigned half = 0; half < 2; ++half) {
        const unsigned base = half * 128;
        for (unsigned l = 0; l < 32; ++l) {
            const unsigned is = l / 16;
            const int q0 = (int)((ql[l] & 0x0fu) | ((qh[l] & 0x03u) << 4)) - 32;
            const int q1 = (int)((ql[l + 32] & 0x0fu) | (((qh[l] >> 2) & 0x03u) << 4)) - 32;
            const int q2 = (int)((ql[l] >> 4) | (((qh[l] >> 4) & 0x03u) << 4)) - 32;
            const int q3 = (int)((ql[l + 32] >> 4) | (((qh[l] >> 6) & 0x03u) << 4)) - 32;
            const int8_t* s = sc + half * 8 + is;
            out[base + l] = d * (float)s[0] * (float)q0;
            out[base + l + 32] = d * (float)s[2] * (float)q1;
            out[base + l + 64] = d * (float)s[4] * (float)q2;
            out[base + l + 96] = d * (float)s[6] * (float)q3;
        }
        ql += 64;
        qh += 32;
    }
}

/* x86 scalar dot_f32 (src/simd_kernels.hpp:12-24): serial, no FMA. */
static float dot_f32(const float* a, const float* b, size_t n) {
    float s = 0.0f;
    for (size_t i = 0; i < n; ++i) s += a[i] * b[i];
    return s;
}

/* x86 scalar dot_i8_f32 (src/simd_kernels.hpp:26-48). */
static float dot_i8_f32(const float* x, const int8_t* q, size_t n) {
    float s = 0.0f;
    for (size_t i = 0; i < n; ++i) s += (float)q[i] * x[i];
    return s;
}

/* unpack_q4_0 scalar branch (src/simd_kernels.hpp:50-65). */
static void unpack_q4_0(const uint8_t* packed, int8_t* out) {
    for (unsigned i = 0; i < 16; ++i) {
        out[i] = (int8_t)((int)(packed[i] & 0x0fu) - 8);
        out[i + 16] = (int8_t)((int)(packed[i] >> 4) - 8);
    }
}

void pko_decode_q4_1(const uint8_t* blk, float* out) {
    const float d = pko_half_to_float(rd16(blk)), m = pko_half_to_float(rd16(blk + 2));
    for (unsigned i = 0; i < 16; ++i) {
        out[i] = (float)(blk[4 + i] & 0x0fu) * d + m;
        out[i + 16] = (float)(blk[4 + i] >> 4) * d + m;
    }
}

static uint32_t rd32(const uint8_t* p) {
    return (uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16) | ((uint32_t)p[3] << 24);
}

/* src/quantized_linear.cpp:64-77: value = fl((q - 16) * d), q = nibble | qh bit << 4,
 * low nibbles first, qh bit i for element i and bit i + 16 for element i + 16. */
void pko_decode_q5_0(const uint8_t* blk, float* out) {
    const float d = pko_half_to_float(rd16(blk));
    const uint32_t qh = rd32(blk + 2);
    for (unsigned i = 0; i < 16; ++i) {
        const int q0 = (int)(blk[6 + i] & 0x0fu) | (int)(((qh >> i) & 1u) << 4);
        const int q1 = (int)(blk[6 + i] >> 4) | (int)(((qh >> (i + 16)) & 1u) << 4);
        out[i] = (float)(q0 - 16) * d;
        out[i + 16] = (float)(q1 - 16) * d;
    }
}

/* src/quantized_linear.cpp:79-93: value = fl(fl(q * d) + m), q unsigned 5-bit. */
void pko_decode_q5_1(const uint8_t* blk, float* out) {
    const float d = pko_half_to_float(rd16(blk)), m = pko_half_to_float(rd16(blk + 2));
    const uint32_t qh = rd32(blk + 4);
    for (unsigned i = 0; i < 16; ++i) {
        const unsigned q0 = (blk[8 + i] & 0x0fu) | (((qh >> i) & 1u) << 4);
        const unsigned q1 = (blk[8 + i] >> 4) | (((qh >> (i + 16)) & 1u) << 4);
        out[i] = (float)q0 * d + m;
        out[i + 16] = (float)q1 * d + m;
    }
}

/* src/quantized_linear.cpp:95-121: 16 scale bytes (low nibble scale, high
 * nibble min), 2-bit quants in 2 chunks of 32 bytes, 4 shifts per chunk, each
 * shift two 16-element groups: value = fl(fl(dl * q) - ml), dl = fl(d * sc),
 * ml = fl(dmin * m); d at 80, dmin at 82. */
void pko_decode_q2_k(const uint8_t* blk, float* out) {
    const float d = pko_half_to_float(rd16(blk + 80)), dmin = pko_half_to_float(rd16(blk + 82));
    const uint8_t* q = blk + 16;
    unsigned si = 0, o = 0;
    for (unsigned chunk = 0; chunk < 2; ++chunk) {
        for (unsigned shift = 0; shift < 8; shift += 2) {
            const uint8_t sc0 = blk[si++], sc1 = blk[si++];
            const float dl0 = d * (float)(sc0 & 0x0fu), ml0 = dmin * (float)(sc0 >> 4);
            const float dl1 = d * (float)(sc1 & 0x0fu), ml1 = dmin * (float)(sc1 >> 4);
            for (unsigned i = 0; i < 16; ++i) out[o++] = dl0 * (float)((q[i] >> shift) & 3u) - ml0;
            for (unsigned i = 0; i < 16; ++i) out[o++] = dl1 * (float)((q[i + 16] >> shift) & 3u) - ml1;
        }
        q += 32;
    }
}

/* src/quantized_linear.cpp:123-164: hmask[32], 2-bit quants in 2 chunks of 32
 * bytes, 12 bytes of packed 6-bit scales (minus 32), d at 108.  value =
 * fl(ds * (q - (hmask bit ? 0 : 4))), ds = fl(d * (scale - 32)). */
void pko_decode_q3_k(const uint8_t* blk, float* out) {
    const uint8_t* hm = blk;
    const uint8_t* q = blk + 32;
    uint32_t aux[4];
    aux[0] = rd32(blk + 96);
    aux[1] = rd32(blk + 100);
    aux[2] = rd32(blk + 104);
    const uint32_t tmp = aux[2];
    aux[2] = ((aux[0] >> 4) & 0x0f0f0f0fu) | (((tmp >> 4) & 0x03030303u) << 4);
    aux[3] = ((aux[1] >> 4) & 0x0f0f0f0fu) | (((tmp >> 6) & 0x03030303u) << 4);
    aux[0] = (aux[0] & 0x0f0f0f0fu) | (((tmp >> 0) & 0x03030303u) << 4);
    aux[1] = (aux[1] & 0x0f0f0f0fu) | (((tmp >> 2) & 0x03030303u) << 4);
    int8_t scales[16];
    memcpy(scales, aux, 16);
    const float d = pko_half_to_float(rd16(blk + 108));
    unsigned si = 0, o = 0;
    unsigned bit = 1;
    for (unsigned chunk = 0; chunk < 2; ++chunk) {
        for (unsigned shift = 0; shift < 8; shift += 2) {
            const float ds0 = d * (float)(scales[si++] - 32);
            const float ds1 = d * (float)(scales[si++] - 32);
            for (unsigned i = 0; i < 16; ++i) {
                const int v = (int)((q[i] >> shift) & 3u) - ((hm[i] & bit) ? 0 : 4);
                out[o++] = ds0 * (float)v;
            }
            for (unsigned i = 0; i < 16; ++i) {
                const int v = (int)((q[i + 16] >> shift) & 3u) - ((hm[i + 16] & bit) ? 0 : 4);
                out[o++] = ds1 * (float)v;
            }
            bit <<= 1;
        }
        q += 32;
    }
}

int pko_dequantize_row(uint32_t type, const uint8_t* enc, uint64_t enc_bytes, float* out,
                       uint64_t count) {
    const uint32_t be = pko_block_elements(type), bb = pko_block_bytes(type);
    if (be < 32 || count == 0 || count % be != 0 || enc_bytes != count / be * bb) return 1;
    const uint64_t blocks = count / be;
    for (uint64_t b = 0; b < blocks; ++b) {
        const uint8_t* blk = enc + b * bb;
        float* row = out + b * be;
        switch (type) {
            case PKO_Q4_0: case PKO_Q8_0: {
                /* src/quantized_linear.cpp:437-449 via scale_i8_f32 (simd_kernels.hpp:85) */
                const float scale = pko_half_to_float(rd16(blk));
                int8_t q[32];
                if (type == PKO_Q4_0) unpack_q4_0(blk + 2, q);
                else memcpy(q, blk + 2, 32);
                for (unsigned i = 0; i < 32; ++i) row[i] = scale * (float)q[i];
                break;
            }
            case PKO_Q4_1: pko_decode_q4_1(blk, row); break;  /* :453-469 */
            case PKO_Q5_0: pko_decode_q5_0(blk, row); break;
            case PKO_Q5_1: pko_decode_q5_1(blk, row); break;
            case PKO_Q2_K: pko_decode_q2_k(blk, row); break;  /* :471-490 */
            case PKO_Q3_K: pko_decode_q3_k(blk, row); break;
            case PKO_Q4_K: pko_decode_q4_k(blk, row); break;
            case PKO_Q5_K: pko_decode_q5_k(blk, row); break;
            case PKO_Q6_K: pko_decode_q6_k(blk, row); break;
            default: return 1;
        }
    }
    return 0;
}

/* Floating rows are converted exactly as TensorReader::read_float_rows_into
 * (src/tensor_reader.cpp:164-198) and fed to linear() (src/linear.cpp:10-31),
 * whose empty bias contributes 0.0F + dot. */
static float float_element(uint32_t type, const uint8_t* row, uint64_t i) {
    if (type == PKO_F32) {
        float f;
        memcpy(&f, row + 4 * i, 4);
        return f;
    }
    if (type == PKO_BF16) return bits_to_float((uint32_t)rd16(row + 2 * i) << 16);
    return pko_half_to_float(rd16(row + 2 * i));
}

int pko_linear(uint32_t type, const uint8_t* w, uint64_t w_bytes, uint64_t in, uint64_t rows,
               const float* x, float* y) {
    const uint32_t be = pko_block_elements(type), bb = pko_block_bytes(type);
    if (be == 0 || in == 0 || rows == 0 || in % be != 0) return 1;
    const uint64_t row_bytes = in / be * bb;
    if (w_bytes != row_bytes * rows) return 1;
    if (be == 1) {
        float* tmp = (float*)malloc(in * sizeof(float));
        if (!tmp) return 2;
        for (uint64_t r = 0; r < rows; ++r) {
            const uint8_t* row = w + r * row_bytes;
            for (uint64_t i = 0; i < in; ++i) tmp[i] = float_element(type, row, i);
            y[r] = 0.0f + dot_f32(tmp, x, in);
        }
        free(tmp);
        return 0;
    }
    const uint64_t blocks = in / be;
    for (uint64_t r = 0; r < rows; ++r) {
        float sum = 0.0f;
        for (uint64_t b = 0; b < blocks; ++b) {
            const uint8_t* blk = w + r * row_bytes + b * bb;
            const float* xb = x + b * be;
            if (type == PKO_Q4_0 || type == PKO_Q8_0) {
                /* linear_quantized (src/quantized_linear.cpp:405-422) */
                const float scale = pko_half_to_float(rd16(blk));
                int8_t q[32];
                if (type == PKO_Q4_0) unpack_q4_0(blk + 2, q);
                else memcpy(q, blk + 2, 32);
                sum += scale * dot_i8_f32(xb, q, 32);
            } else if (be == 32) {
                /* linear_k<32, 20/22/24> with decode_q4_1 / q5_0 / q5_1
                 * (src/quantized_linear.cpp:503-519) */
                float dec[32];
                if (type == PKO_Q4_1) pko_decode_q4_1(blk, dec);
                else if (type == PKO_Q5_0) pko_decode_q5_0(blk, dec);
                else pko_decode_q5_1(blk, dec);
                sum += dot_f32(dec, xb, 32);
            } else {
                /* linear_k (src/quantized_linear.cpp:374-384) for Q2_K..Q6_K
                 * (:529-561); on x86 Q4_K takes this decode-then-dot branch
                 * (:541-549). */
                float dec[256];
                if (type == PKO_Q2_K) pko_decode_q2_k(blk, dec);
                else if (type == PKO_Q3_K) pko_decode_q3_k(blk, dec);
                else if (type == PKO_Q4_K) pko_decode_q4_k(blk, dec);
                else if (type == PKO_Q5_K) pko_decode_q5_k(blk, dec);
                else pko_decode_q6_k(blk, dec);
                sum += dot_f32(dec, xb, 256);
            }
        }
        y[r] = sum;
    }
    return 0;
}

/* src/qwen3_moe_runner.cpp:267-305 */
int pko_route_experts(const float* logits, uint32_t n, uint32_t top_k, int normalize,
                      uint32_t* ids, float* sel_logits, float* probs) {
    if (top_k == 0 || top_k > n) return 1;
    /* std::max_element: first maximum under operator< */
    uint32_t mi = 0;
    for (uint32_t i = 1; i < n; ++i)
        if (logits[mi] < logits[i]) mi = i;
    const float mx = logits[mi];
    if (!isfinite(mx)) return 2;
    for (uint32_t i = 0; i < n; ++i)
        if (!isfinite(logits[i])) return 2;
    double denominator = 0.0;
    for (uint32_t i = 0; i < n; ++i) denominator += exp((double)(logits[i] - mx));
    /* sorted insertion by (logit desc, id asc); keep the first top_k */
    uint32_t count = 0;
    for (uint32_t id = 0; id < n; ++id) {
        const float v = logits[id];
        uint32_t where = 0;
        while (where < count && (logits[ids[where]] > v ||
                                 (logits[ids[where]] == v && ids[where] < id)))
            ++where;
        if (count < top_k) {
            for (uint32_t j = count; j > where; --j) ids[j] = ids[j - 1];
            ids[where] = id;
            ++count;
        } else if (where < count) {
            for (uint32_t j = count - 1; j > where; --j) ids[j] = ids[j - 1];
            ids[where] = id;
        }
    }
    float selected_sum = 0.0f;
    for (uint32_t i = 0; i < top_k; ++i) {
        const uint32_t id = ids[i];
        probs[i] = (float)(exp((double)(logits[id] - mx)) / denominator);
        selected_sum += probs[i];
        if (sel_logits) sel_logits[i] = logits[id];
    }
    if (normalize)
        for (uint32_t i = 0; i < top_k; ++i) probs[i] /= selected_sum;
    return 0;
}

/* src/qwen3_moe_runner.cpp:643-692 (rms_norm at :643 and the residual add at
 * :692 are the caller's). */
int pko_moe_block(const float* router, uint32_t hidden, uint32_t n_experts, uint32_t ffn,
                  uint32_t gate_type, const uint8_t* gate, uint32_t up_type, const uint8_t* up,
                  uint32_t down_type, const uint8_t* down, uint32_t top_k, int normalize,
                  const float* x, float* y, uint32_t* ids, float* probs) {
    if (hidden == 0 || n_experts == 0 || ffn == 0 || top_k == 0 || top_k > n_experts) return 1;
    const uint64_t gate_be = pko_block_elements(gate_type), up_be = pko_block_elements(up_type),
                   down_be = pko_block_elements(down_type);
    if (!gate_be || !up_be || !down_be || hidden % gate_be || hidden % up_be || ffn % down_be)
        return 1;
    const uint64_t gate_slice = (uint64_t)ffn * (hidden / gate_be) * pko_block_bytes(gate_type);
    const uint64_t up_slice = (uint64_t)ffn * (hidden / up_be) * pko_block_bytes(up_type);
    const uint64_t down_slice = (uint64_t)hidden * (ffn / down_be) * pko_block_bytes(down_type);
    float* logits = (float*)malloc(sizeof(float) * n_experts);
    float* g = (float*)malloc(sizeof(float) * ffn);
    float* u = (float*)malloc(sizeof(float) * ffn);
    float* act = (float*)malloc(sizeof(float) * ffn);
    float* out = (float*)malloc(sizeof(float) * hidden);
    int rc = 2;
    if (!logits || !g || !u || !act || !out) goto done;
    rc = pko_linear(PKO_F32, (const uint8_t*)router, (uint64_t)hidden * n_experts * 4, hidden,
                    n_experts, x, logits);
    if (rc) goto done;
    rc = pko_route_experts(logits, n_experts, top_k, normalize, ids, NULL, probs);
    if (rc) goto done;
    for (uint32_t i = 0; i < hidden; ++i) y[i] = 0.0f;
    for (uint32_t r = 0; r < top_k; ++r) {
        const uint64_t e = ids[r];
        rc = pko_linear(gate_type, gate + e * gate_slice, gate_slice, hidden, ffn, x, g);
        if (!rc) rc = pko_linear(up_type, up + e * up_slice, up_slice, hidden, ffn, x, u);
        if (rc) goto done;
        for (uint32_t i = 0; i < ffn; ++i) act[i] = (g[i] / (1.0f + expf(-g[i]))) * u[i];
        rc = pko_linear(down_type, down + e * down_slice, down_slice, ffn, hidden, act, out);
        if (rc) goto done;
        for (uint32_t i = 0; i < hidden; ++i) y[i] += probs[r] * out[i];
    }
    rc = 0;
done:
    free(logits);
    free(g);
    free(u);
    free(act);
    free(out);
    return rc;
}

/* src/qwen35_runner.cpp:131-173 */
int pko_select_experts(const float* logits, uint32_t n, uint32_t top_k, int normalize,
                       uint32_t* ids, float* weights) {
    if (top_k == 0 || top_k > n) return 1;
    float mx = logits[0];
    for (uint32_t i = 1; i < n; ++i)
        if (mx < logits[i]) mx = logits[i];
    if (!isfinite(mx)) return 2;
    for (uint32_t i = 0; i < n; ++i)
        if (!isfinite(logits[i])) return 2;
    float* prob = (float*)malloc(sizeof(float) * n);
    if (!prob) return 2;
    float denominator = 0.0f;
    for (uint32_t i = 0; i < n; ++i) {
        prob[i] = expf(logits[i] - mx);
        denominator += prob[i];
    }
    if (!isfinite(denominator) || denominator <= 0.0f) {
        free(prob);
        return 2;
    }
    for (uint32_t i = 0; i < n; ++i) prob[i] /= denominator;
    uint32_t count = 0;
    for (uint32_t id = 0; id < n; ++id) {
        const float v = logits[id];
        uint32_t where = 0;
        while (where < count && (logits[ids[where]] > v ||
                                 (logits[ids[where]] == v && ids[where] < id)))
            ++where;
        if (count < top_k) {
            for (uint32_t j = count; j > where; --j) ids[j] = ids[j - 1];
            ids[where] = id;
            ++count;
        } else if (where < count) {
            for (uint32_t j = count - 1; j > where; --j) ids[j] = ids[j - 1];
            ids[where] = id;
        }
    }
    for (uint32_t i = 0; i < top_k; ++i) weights[i] = prob[ids[i]];
    free(prob);
    if (normalize) {
        float sum = 0.0f;
        for (uint32_t i = 0; i < top_k; ++i) sum += weights[i];
        if (!isfinite(sum) || sum <= 0.0f) return 2;
        for (uint32_t i = 0; i < top_k; ++i) weights[i] /= sum;
    }
    return 0;
}

/* src/qwen35_runner.cpp:111-115 and :123 */
static float pko_sigmoid35(float v) {
    if (v >= 0.0f) return 1.0f / (1.0f + expf(-v));
    const float e = expf(v);
    return e / (1.0f + e);
}

static int pko_ffn_silu(uint32_t gate_type, const uint8_t* gate, uint64_t gate_bytes,
                        uint32_t up_type, const uint8_t* up, uint64_t up_bytes, uint32_t down_type,
                        const uint8_t* down, uint64_t down_bytes, uint32_t hidden, uint32_t ffn,
                        const float* x, float* g, float* u, float* act, float* out) {
    int rc = pko_linear(gate_type, gate, gate_bytes, hidden, ffn, x, g);
    if (!rc) rc = pko_linear(up_type, up, up_bytes, hidden, ffn, x, u);
    if (rc) return rc;
    for (uint32_t i = 0; i < ffn; ++i) act[i] = (g[i] * pko_sigmoid35(g[i])) * u[i];
    return pko_linear(down_type, down, down_bytes, ffn, hidden, act, out);
}

/* src/qwen35_runner.cpp:690-761 (the norm before and the residual add after
 * are the caller's). */
int pko_moe35_block(const float* router, uint32_t hidden, uint32_t n_experts, uint32_t ffn,
                    uint32_t gate_type, const uint8_t* gate, uint32_t up_type, const uint8_t* up,
                    uint32_t down_type, const uint8_t* down, uint32_t top_k, int normalize,
                    float scale, const float* shared_router, uint32_t shared_ffn,
                    uint32_t sgate_type, const uint8_t* sgate, uint32_t sup_type,
                    const uint8_t* sup, uint32_t sdown_type, const uint8_t* sdown,
                    const float* x, float* y, uint32_t* ids, float* weights) {
    if (hidden == 0 || n_experts == 0 || ffn == 0 || shared_ffn == 0 || top_k == 0 ||
        top_k > n_experts)
        return 1;
    const uint32_t types[6] = {gate_type, up_type, down_type, sgate_type, sup_type, sdown_type};
    const uint32_t ins[6] = {hidden, hidden, ffn, hidden, hidden, shared_ffn};
    for (int i = 0; i < 6; ++i) {
        const uint64_t be = pko_block_elements(types[i]);
        if (!be || ins[i] % be) return 1;
    }
    const uint64_t gate_slice = (uint64_t)ffn * (hidden / pko_block_elements(gate_type)) * pko_block_bytes(gate_type);
    const uint64_t up_slice = (uint64_t)ffn * (hidden / pko_block_elements(up_type)) * pko_block_bytes(up_type);
    const uint64_t down_slice = (uint64_t)hidden * (ffn / pko_block_elements(down_type)) * pko_block_bytes(down_type);
    const uint64_t sg_bytes = (uint64_t)shared_ffn * (hidden / pko_block_elements(sgate_type)) * pko_block_bytes(sgate_type);
    const uint64_t su_bytes = (uint64_t)shared_ffn * (hidden / pko_block_elements(sup_type)) * pko_block_bytes(sup_type);
    const uint64_t sd_bytes = (uint64_t)hidden * (shared_ffn / pko_block_elements(sdown_type)) * pko_block_bytes(sdown_type);
    const uint32_t wmax = ffn > shared_ffn ? ffn : shared_ffn;
    float* logits = (float*)malloc(sizeof(float) * n_experts);
    float* g = (float*)malloc(sizeof(float) * wmax);
    float* u = (float*)malloc(sizeof(float) * wmax);
    float* act = (float*)malloc(sizeof(float) * wmax);
    float* out = (float*)malloc(sizeof(float) * hidden);
    float gate_value = 0.0f;
    int rc = 2;
    if (!logits || !g || !u || !act || !out) goto done;
    rc = pko_linear(PKO_F32, (const uint8_t*)router, (uint64_t)hidden * n_experts * 4, hidden,
                    n_experts, x, logits);
    if (!rc) rc = pko_select_experts(logits, n_experts, top_k, normalize, ids, weights);
    if (rc) goto done;
    for (uint32_t i = 0; i < hidden; ++i) y[i] = 0.0f;
    for (uint32_t r = 0; r < top_k; ++r) {
        const uint64_t e = ids[r];
        rc = pko_ffn_silu(gate_type, gate + e * gate_slice, gate_slice, up_type, up + e * up_slice,
                          up_slice, down_type, down + e * down_slice, down_slice, hidden, ffn, x,
                          g, u, act, out);
        if (rc) goto done;
        const float route_scale = weights[r] * scale;
        for (uint32_t i = 0; i < hidden; ++i) y[i] += route_scale * out[i];
    }
    rc = pko_linear(PKO_F32, (const uint8_t*)shared_router, (uint64_t)hidden * 4, hidden, 1, x,
                    &gate_value);
    if (!rc)
        rc = pko_ffn_silu(sgate_type, sgate, sg_bytes, sup_type, sup, su_bytes, sdown_type, sdown,
                          sd_bytes, hidden, shared_ffn, x, g, u, act, out);
    if (rc) goto done;
    {
        const float shared_scale = pko_sigmoid35(gate_value);
        for (uint32_t i = 0; i < hidden; ++i) y[i] = y[i] + shared_scale * out[i];
    }
    rc = 0;
done:
    free(logits);
    free(g);
    free(u);
    free(act);
    free(out);
    return rc;
}


/* ---- the host libm's expf as block checksums ---------------------------------- */

typedef struct {
    uint32_t first_bits, block_size, k0, k1;
    uint64_t* sums;
} ExpfJob;

static void* expf_job(void* arg) {
    const ExpfJob* j = (const ExpfJob*)arg;
    for (uint32_t k = j->k0; k < j->k1; ++k) {
        uint64_t acc = 0;
        const uint32_t base = j->first_bits + k * j->block_size;
        for (uint32_t i = 0; i < j->block_size; ++i) {
            const uint32_t b = base + i;
            float x, r;
            memcpy(&x, &b, 4);
            r = expf(x);
            uint32_t rb;
            memcpy(&rb, &r, 4);
            acc += (((uint64_t)rb << 32) | b) * 0xD6E8FEB86659FD93ull;
        }
        j->sums[k] = acc;
    }
    return NULL;
}

void pko_expf_block_sums(uint32_t first_bits, uint32_t block_size, uint32_t n_blocks,
                         uint64_t* sums, uint32_t threads) {
    if (threads == 0) threads = 1;
    if (threads > 64) threads = 64;
    pthread_t th[64];
    int created[64] = {0};
    ExpfJob jobs[64];
    const uint32_t per = (n_blocks + threads - 1) / threads;
    for (uint32_t t = 0; t < threads; ++t) {
        const uint32_t k0 = t * per, k1 = k0 + per < n_blocks ? k0 + per : n_blocks;
        if (k0 >= k1) break;
        jobs[t] = (ExpfJob){first_bits, block_size, k0, k1, sums};
        created[t] = pthread_create(&th[t], NULL, expf_job, &jobs[t]) == 0;
        if (!created[t]) expf_job(&jobs[t]);  /* inline when a thread cannot start */
    }
    for (uint32_t t = 0; t < threads; ++t)
        if (created[t]) pthread_join(th[t], NULL);
}

/* rms_norm (src/rms_norm.cpp:9-27): sum_squares = dot_f32(x, x, n), the serial
 * unfused chain of src/simd_kernels.hpp:12-24 (x86 branch); mean = sum / n;
 * scale = 1 / sqrt(mean + eps); out_i = (x_i * scale) * w_i
 * (rms_scale_f32, simd_kernels.hpp:109-122).  Rows of n values, row-major. */
int pko_rms_norm(const float* x, const float* w, uint64_t rows, uint64_t n, float eps,
                 float* out) {
    if (!x || !w || !out || n == 0) return 1;
    for (uint64_t r = 0; r < rows; ++r) {
        const float* xr = x + r * n;
        float* o = out + r * n;
        float sum = 0.0f;
        for (uint64_t i = 0; i < n; ++i) sum += xr[i] * xr[i];
        const float mean = sum / (float)n;
        const float scale = 1.0f / sqrtf(mean + eps);
        for (uint64_t i = 0; i < n; ++i) o[i] = xr[i] * scale * w[i];
    }
    return 0;
}

/* float_to_half of src/kv_cache.cpp:20-44: binary32 -> binary16, round to
 * nearest even, NaN kept quiet with payload 0x200, overflow to infinity. */
static uint16_t float_to_half_rne(float value) {
    uint32_t bits;
    memcpy(&bits, &value, 4);
    const uint16_t sign = (uint16_t)((bits >> 16) & 0x8000u);
    const uint32_t exponent = (bits >> 23) & 0xffu;
    uint32_t mantissa = bits & 0x7fffffu;
    if (exponent == 0xffu) return (uint16_t)(sign | 0x7c00u | (mantissa ? 0x0200u : 0u));
    int half_exponent = (int)exponent - 127 + 15;
    if (half_exponent >= 31) return (uint16_t)(sign | 0x7c00u);
    if (half_exponent <= 0) {
        if (half_exponent < -10) return sign;
        mantissa |= 0x800000u;
        const unsigned shift = (unsigned)(14 - half_exponent);
        const uint32_t rounding = (1u << (shift - 1)) - 1u + ((mantissa >> shift) & 1u);
        return (uint16_t)(sign | ((mantissa + rounding) >> shift));
    }
    mantissa += 0x0fffu + ((mantissa >> 13) & 1u);
    if (mantissa & 0x800000u) {
        mantissa = 0;
        if (++half_exponent >= 31) return (uint16_t)(sign | 0x7c00u);
    }
    return (uint16_t)(sign | ((uint16_t)half_exponent << 10) | (uint16_t)(mantissa >> 13));
}

/* One layer's attention for positions 0 .. steps - 1, as the runner's token
 * step does it (src/qwen3_moe_runner.cpp:610-628): rms_norm of every q and k
 * head with the head norm weights (src/rms_norm.cpp:9-27), NeoX RoPE with the
 * angles of prepare_qwen_rope (:141-155: angle = pos * powf(theta, -p / half),
 * cosf, sinf) applied as rope_rotate_f32 (src/simd_kernels.hpp:88-108: a' = a c
 * - b s, b' = b c + a s over the two halves), KvCache::append in FP16
 * (src/kv_cache.cpp:131-168) and KvCache::attend (:170-294): per q head the
 * serial dot with each cached key (decoded from FP16) times 1/sqrt(head_dim),
 * the maximum, expf(score - max) and their serial sum in window order, then
 * out += (score / sum) * value in window order.  The ring holds the last
 * `capacity` positions.  q[t] [heads][head_dim], k[t] / v[t] [kv_heads][head_dim]
 * are step t's projections before the head norms; out[t] [heads][head_dim]. */
int pko_attention_steps(uint32_t heads, uint32_t kv_heads, uint32_t head_dim, uint32_t capacity,
                        float eps, float theta, const float* q_norm, const float* k_norm,
                        uint32_t steps, const float* q, const float* k, const float* v,
                        float* out) {
    if (!heads || !kv_heads || heads % kv_heads || !head_dim || head_dim % 2 || !capacity ||
        !q_norm || !k_norm || !q || !k || !v || !out)
        return 1;
    const uint32_t half = head_dim / 2, group = heads / kv_heads;
    const uint64_t qd = (uint64_t)heads * head_dim, kd = (uint64_t)kv_heads * head_dim;
    uint16_t* kc = (uint16_t*)malloc(sizeof(uint16_t) * capacity * kd);
    uint16_t* vc = (uint16_t*)malloc(sizeof(uint16_t) * capacity * kd);
    float* qq = (float*)malloc(sizeof(float) * qd);
    float* kk = (float*)malloc(sizeof(float) * kd);
    float* cs = (float*)malloc(sizeof(float) * head_dim);
    float* key = (float*)malloc(sizeof(float) * head_dim);
    float* val = (float*)malloc(sizeof(float) * head_dim);
    float* sc = (float*)malloc(sizeof(float) * (uint64_t)capacity * group);
    float* mx = (float*)malloc(sizeof(float) * group);
    float* den = (float*)malloc(sizeof(float) * group);
    int rc = (kc && vc && qq && kk && cs && key && val && sc && mx && den) ? 0 : 2;
    const float scale = 1.0f / sqrtf((float)head_dim);
    for (uint32_t t = 0; t < steps && !rc; ++t) {
        memcpy(qq, q + t * qd, sizeof(float) * qd);
        memcpy(kk, k + t * kd, sizeof(float) * kd);
        for (uint32_t h = 0; h < heads; ++h) pko_rms_norm(qq + h * head_dim, q_norm, 1, head_dim, eps, qq + h * head_dim);
        for (uint32_t h = 0; h < kv_heads; ++h) pko_rms_norm(kk + h * head_dim, k_norm, 1, head_dim, eps, kk + h * head_dim);
        for (uint32_t p = 0; p < half; ++p) {
            const float angle = (float)t * powf(theta, -(float)p / (float)half);
            cs[p] = cosf(angle);
            cs[half + p] = sinf(angle);
        }
        for (uint32_t h = 0; h < heads + kv_heads; ++h) {
            float* vec = h < heads ? qq + h * head_dim : kk + (h - heads) * head_dim;
            for (uint32_t i = 0; i < half; ++i) {
                const float a = vec[i], b = vec[half + i];
                vec[i] = a * cs[i] - b * cs[half + i];
                vec[half + i] = b * cs[i] + a * cs[half + i];
            }
        }
        const uint32_t slot_now = t % capacity;
        for (uint64_t i = 0; i < kd; ++i) {
            kc[slot_now * kd + i] = float_to_half_rne(kk[i]);
            vc[slot_now * kd + i] = float_to_half_rne(v[t * kd + i]);
        }
        const uint32_t size = t + 1 < capacity ? t + 1 : capacity, first = t + 1 - size;
        for (uint32_t kh = 0; kh < kv_heads; ++kh) {
            for (uint32_t g = 0; g < group; ++g) mx[g] = -INFINITY;
            for (uint32_t i = 0; i < size; ++i) {
                const uint32_t slot = (first + i) % capacity;
                for (uint32_t d = 0; d < head_dim; ++d) key[d] = pko_half_to_float(kc[slot * kd + kh * head_dim + d]);
                for (uint32_t g = 0; g < group; ++g) {
                    float s = dot_f32(qq + (kh * group + g) * head_dim, key, head_dim);
                    s *= scale;
                    sc[g * capacity + i] = s;
                    mx[g] = mx[g] < s ? s : mx[g];  /* std::max(current, score) */
                }
            }
            for (uint32_t g = 0; g < group; ++g) {
                float sum = 0.0f;
                for (uint32_t i = 0; i < size; ++i) {
                    float* s = sc + g * capacity + i;
                    *s = expf(*s - mx[g]);
                    sum += *s;
                }
                den[g] = sum;
                memset(out + t * qd + (kh * group + g) * head_dim, 0, sizeof(float) * head_dim);
            }
            for (uint32_t i = 0; i < size; ++i) {
                const uint32_t slot = (first + i) % capacity;
                for (uint32_t d = 0; d < head_dim; ++d) val[d] = pko_half_to_float(vc[slot * kd + kh * head_dim + d]);
                for (uint32_t g = 0; g < group; ++g) {
                    const float prob = sc[g * capacity + i] / den[g];
                    float* o = out + t * qd + (kh * group + g) * head_dim;
                    for (uint32_t d = 0; d < head_dim; ++d) o[d] += prob * val[d];
                }
            }
        }
    }
    free(kc); free(vc); free(qq); free(kk); free(cs); free(key); free(val); free(sc); free(mx); free(den);
    return rc;
}

/* The fast decode's residual add and RMSNorm as the reference runner does
 * them (src/qwen3_moe_runner.cpp:630,692 then src/rms_norm.cpp:9-27):
 * hidden_i += delta_i (FP32), then out = rms_norm(hidden, w, eps).  Rows of
 * n values; delta may be null (no add). */
int pko_add_rms_norm(float* hidden, const float* delta, const float* w, uint64_t rows, uint64_t n,
                     float eps, float* out) {
    if (!hidden || !w || !out || n == 0) return 1;
    if (delta)
        for (uint64_t i = 0; i < rows * n; ++i) hidden[i] += delta[i];
    return pko_rms_norm(hidden, w, rows, n, eps, out);
}
