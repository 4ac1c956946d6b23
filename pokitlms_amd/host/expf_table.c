/* expf_table.c -- writes the table of float inputs on which this host's libm
 * expf differs from the correctly rounded exp (exp in double, rounded once to
 * float), with libm's result for each.
 *
 * The reference CPU path computes its softmax and SwiGLU exponentials with
 * the host libm's expf (src/kv_cache.cpp:249, src/qwen3_moe_runner.cpp:683).
 * The device computes the correctly rounded value and, in the reference-order
 * decode, replaces it by the entry found here, so both give the same bits.
 *
 * Output (little endian): "PKEXPF01", uint32 count, then count pairs
 * (uint32 input bits, uint32 result bits) in increasing input-bit order.
 * Usage: expf_table <output file>
 */
#include <math.h>
#include <pthread.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#define THREADS 8

typedef struct {
    uint32_t lo, hi;  /* input-bit range [lo, hi) */
    uint32_t* pairs;
    size_t count, cap;
} Slice;

static void* scan(void* arg) {
    Slice* s = (Slice*)arg;
    for (uint64_t u = s->lo; u < s->hi; ++u) {
        const uint32_t bits = (uint32_t)u;
        float x;
        memcpy(&x, &bits, 4);
        if (!isfinite(x)) continue;
        const float got = expf(x);
        const float cr = (float)exp((double)x);
        uint32_t gb, cb;
        memcpy(&gb, &got, 4);
        memcpy(&cb, &cr, 4);
        if (gb == cb) continue;
        if (s->count == s->cap) {
            s->cap = s->cap ? 2 * s->cap : 4096;
            s->pairs = (uint32_t*)realloc(s->pairs, 2 * s->cap * sizeof(uint32_t));
            if (!s->pairs) return (void*)1;
        }
        s->pairs[2 * s->count] = bits;
        s->pairs[2 * s->count + 1] = gb;
        ++s->count;
    }
    return NULL;
}

int main(int argc, char** argv) {
    if (argc != 2) {
        fprintf(stderr, "usage: %s <output>\n", argv[0]);
        return 2;
    }
    Slice slices[THREADS];
    pthread_t th[THREADS];
    const uint64_t span = (1ull << 32) / THREADS;
    for (int t = 0; t < THREADS; ++t) {
        memset(&slices[t], 0, sizeof(Slice));
        slices[t].lo = (uint32_t)(t * span);
        slices[t].hi = t + 1 == THREADS ? 0xffffffffu : (uint32_t)((t + 1) * span);
        pthread_create(&th[t], NULL, scan, &slices[t]);
    }
    size_t total = 0;
    for (int t = 0; t < THREADS; ++t) {
        void* rc = NULL;
        pthread_join(th[t], &rc);
        if (rc) return 1;
        total += slices[t].count;
    }
    FILE* f = fopen(argv[1], "wb");
    if (!f) return 1;
    const uint32_t n = (uint32_t)total;
    fwrite("PKEXPF01", 1, 8, f);
    fwrite(&n, 4, 1, f);
    for (int t = 0; t < THREADS; ++t) fwrite(slices[t].pairs, 8, slices[t].count, f);
    fclose(f);
    printf("%u entries\n", n);
    return 0;
}
