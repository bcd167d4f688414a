/* CPU restatement of bc-infer's sampler (crates/bc-infer/src/sample.rs): TEST INFRASTRUCTURE,
 * NOT PRODUCT CODE. Only tests/ use it, as the checker of the GPU sampler (bchip_sample). Built
 * with -ffp-contract=off: every sum, quotient and product rounds on its own, as the reference's
 * Rust does.
 *
 * One choice the reference leaves to its platform: f32::exp calls the C library's expf, whose
 * last bit may differ between libraries (glibc's has a 0.502-ulp bound, and an FMA variant
 * chosen at run time). Here exp is the correctly rounded f32 value, computed as
 * (float)exp((double)x); the GPU sampler computes the same. It equals glibc's expf except for
 * arguments within 0.002 ulp of a rounding midpoint. */
#include "bc_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

/* sample.rs:24-32: the first index of the highest score (strict >, so a NaN never wins past
 * index 0). */
uint32_t bcs_argmax(const float* s, uint32_t n) {
    uint32_t best = 0;
    for (uint32_t i = 0; i < n; i++)
        if (s[i] > s[best]) best = i;
    return best;
}

/* sample.rs:74-81: splitmix64 one step from the seed, the top 24 bits over 2^24. */
float bcs_uniform(uint64_t seed) {
    uint64_t z = seed + 0x9e3779b97f4a7c15ull;
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
    z ^= z >> 31;
    return (float)(z >> 40) / (float)(1ull << 24);
}

float bcs_exp(float x) { return (float)exp((double)x); }

/* f32::total_cmp as an unsigned key: ascending keys are ascending total order (-NaN < -inf <
 * ... < -0 < +0 < ... < +inf < +NaN). */
static uint32_t total_key(float x) {
    uint32_t b;
    memcpy(&b, &x, 4);
    return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

typedef struct {
    uint32_t id;
    float w;
} bcs_pair;

/* Descending total order, the earlier index first among equals: slice::sort_by is stable. */
static int by_weight(const void* a, const void* b) {
    const bcs_pair* x = (const bcs_pair*)a;
    const bcs_pair* y = (const bcs_pair*)b;
    uint32_t kx = total_key(x->w), ky = total_key(y->w);
    if (kx != ky) return kx > ky ? -1 : 1;
    return x->id < y->id ? -1 : (x->id > y->id ? 1 : 0);
}

/* sample.rs:35-71. */
uint32_t bcs_sample(const float* scores, uint32_t n, float temperature, float top_p, uint64_t seed,
                    uint64_t step) {
    if (!(temperature > 0.0f)) return bcs_argmax(scores, n);
    float max = -INFINITY;
    for (uint32_t i = 0; i < n; i++) max = fmaxf(max, scores[i]); /* f32::max skips NaN */
    bcs_pair* p = (bcs_pair*)malloc(sizeof(bcs_pair) * n);
    for (uint32_t i = 0; i < n; i++) {
        p[i].id = i;
        p[i].w = bcs_exp((scores[i] - max) / temperature);
    }
    float total = -0.0f; /* Iterator::sum over f32 */
    for (uint32_t i = 0; i < n; i++) total += p[i].w;
    qsort(p, n, sizeof(bcs_pair), by_weight);
    uint32_t keep = 0;
    float mass = 0.0f;
    for (uint32_t i = 0; i < n; i++) {
        keep++;
        mass += p[i].w / total;
        if (mass >= top_p) break;
    }
    if (keep < 1) keep = 1;
    float kept = -0.0f;
    for (uint32_t i = 0; i < keep; i++) kept += p[i].w;
    float r = bcs_uniform(seed ^ (step * 0x9e3779b97f4a7c15ull)) * kept;
    uint32_t id = p[0].id;
    for (uint32_t i = 0; i < keep; i++) {
        r -= p[i].w;
        if (r <= 0.0f) {
            id = p[i].id;
            break;
        }
    }
    free(p);
    return id;
}
