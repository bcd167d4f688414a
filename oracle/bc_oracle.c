/* CPU oracle for bc-infer's attention path: TEST INFRASTRUCTURE, NOT PRODUCT CODE.
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg use it, as the
 * checker; the product library never does. Built with -ffp-contract=off so that every
 * product and sum rounds separately, as the reference's Rust (which never contracts to
 * FMA) does. Reference citations are per function; see bc_oracle.h. */
#include "bc_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

/* model.rs:208-211: base.powf(-2.0 * i as f32 / rope_dim as f32) / factor, all in f32. */
void bco_inv_freq(float* out, uint32_t rope_dim, float base, const float* factors) {
    for (uint32_t i = 0; i < rope_dim / 2; i++) {
        float e = -2.0f * (float)i / (float)rope_dim;
        float f = factors ? factors[i] : 1.0f;
        out[i] = powf(base, e) / f;
    }
}

/* model.rs:391-403. theta = pos as f32 * inv_freq[i]; (sin, cos) in f32; neox pairs
 * (i, i + half), else (2i, 2i + 1). */
void bco_rope(float* x, uint32_t heads, uint32_t head_dim, uint32_t rope_dim, int neox,
              uint64_t pos, const float* inv_freq) {
    uint32_t half = rope_dim / 2;
    for (uint32_t h = 0; h < heads; h++) {
        float* head = x + (size_t)h * head_dim;
        for (uint32_t i = 0; i < half; i++) {
            float theta = (float)pos * inv_freq[i];
            float s = sinf(theta), c = cosf(theta);
            uint32_t a = neox ? i : 2 * i;
            uint32_t b = neox ? i + half : 2 * i + 1;
            float x0 = head[a], x1 = head[b];
            head[a] = x0 * c - x1 * s;
            head[b] = x0 * s + x1 * c;
        }
    }
}

/* model.rs:421-443 (Shape::new). */
int bco_shape(uint32_t rows, uint64_t pos, const uint32_t* tree, uint32_t tree_len,
              uint64_t* positions, uint64_t* visible, uint64_t* base) {
    if (!tree) {
        for (uint32_t i = 0; i < rows; i++) positions[i] = pos + i;
        if (base) *base = pos;
        return 0;
    }
    if (tree_len < rows || tree_len > BCO_MAX_TREE || (uint64_t)(tree_len - rows) > pos) return -1;
    uint64_t b = pos + rows - tree_len;
    uint64_t pp[BCO_MAX_TREE], vv[BCO_MAX_TREE];
    for (uint32_t i = 0; i < tree_len; i++) {
        uint32_t p = tree[i];
        uint64_t depth, seen;
        if (p == BCO_ROOT) {
            depth = 0;
            seen = 0;
        } else if (p < i) {
            depth = pp[p] - b + 1;
            seen = vv[p];
        } else {
            return -1;
        }
        pp[i] = b + depth;
        vv[i] = seen | (1ull << i);
    }
    uint32_t skip = tree_len - rows;
    for (uint32_t i = 0; i < rows; i++) {
        positions[i] = pp[skip + i];
        if (visible) visible[i] = vv[skip + i];
    }
    if (base) *base = b;
    return 0;
}

/* quant.rs:617-631: eight lane sums over whole chunks of 8, summed lane 0..7 from zero,
 * then the remainder added in order. */
float bco_dot(const float* a, const float* b, size_t n) {
    float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    size_t whole = n / 8 * 8;
    for (size_t c = 0; c < whole; c += 8)
        for (int k = 0; k < 8; k++) acc[k] += a[c + k] * b[c + k];
    float sum = 0.0f;
    for (int k = 0; k < 8; k++) sum += acc[k];
    for (size_t i = whole; i < n; i++) sum += a[i] * b[i];
    return sum;
}

/* model.rs:448-481. Per row: the visible slot list (line: 0..pos+i+1; tree: 0..base then
 * base+j for each set bit j < pos+rows-base); per head: scores = dot*scale, max, exp(s-max)
 * summed in slot order, then o += (p/sum)*v in slot order. kvh = h / (nh/nkv). */
void bco_attention(const float* q, const float* kc, const float* vc, float* out,
                   uint32_t rows, uint64_t pos, const uint64_t* visible, uint64_t base,
                   uint32_t nh, uint32_t nkv, uint32_t hd, float scale) {
    size_t kvd = (size_t)nkv * hd;
    uint32_t group = nh / (nkv ? nkv : 1);
    if (group == 0) group = 1;
    size_t most = pos + rows;
    uint64_t* slots = (uint64_t*)malloc(sizeof(uint64_t) * (most + 1));
    float* scores = (float*)malloc(sizeof(float) * (most + 1));
    memset(out, 0, sizeof(float) * (size_t)rows * nh * hd);
    for (uint32_t i = 0; i < rows; i++) {
        size_t n = 0;
        if (!visible) {
            for (uint64_t t = 0; t < pos + i + 1; t++) slots[n++] = t;
        } else {
            for (uint64_t t = 0; t < base; t++) slots[n++] = t;
            for (uint64_t j = 0; j < pos + rows - base; j++)
                if ((visible[i] >> j) & 1ull) slots[n++] = base + j;
        }
        for (uint32_t h = 0; h < nh; h++) {
            const float* qh = q + ((size_t)i * nh + h) * hd;
            uint32_t kvh = h / group;
            float mx = -INFINITY;
            for (size_t s = 0; s < n; s++) {
                scores[s] = bco_dot(qh, kc + slots[s] * kvd + (size_t)kvh * hd, hd) * scale;
                if (scores[s] > mx) mx = scores[s];
            }
            float sum = 0.0f;
            for (size_t s = 0; s < n; s++) {
                scores[s] = expf(scores[s] - mx);
                sum += scores[s];
            }
            float* o = out + ((size_t)i * nh + h) * hd;
            for (size_t s = 0; s < n; s++) {
                const float* vt = vc + slots[s] * kvd + (size_t)kvh * hd;
                float w = scores[s] / sum;
                for (uint32_t d = 0; d < hd; d++) o[d] += w * vt[d];
            }
        }
    }
    free(slots);
    free(scores);
}

/* model.rs:146-166 (Kv::keep), for one cache buffer. */
int bco_keep(float* cache, uint64_t width, uint64_t* len, uint64_t base,
             const uint32_t* rows, uint32_t nrows) {
    for (uint32_t n = 0; n + 1 < nrows; n++)
        if (rows[n] >= rows[n + 1]) return -1;
    for (uint32_t n = 0; n < nrows; n++)
        if (base + rows[n] >= *len) return -1;
    for (uint32_t n = 0; n < nrows; n++) {
        uint64_t from = (base + rows[n]) * width, to = (base + n) * width;
        memmove(cache + to, cache + from, sizeof(float) * width);
    }
    *len = base + nrows;
    return 0;
}

/* IEEE binary16 round to nearest even, with subnormals, infinities and NaN. */
uint16_t bco_f32_to_f16(float x) {
    uint32_t b;
    memcpy(&b, &x, 4);
    uint32_t sign = (b >> 16) & 0x8000u;
    uint32_t exp = (b >> 23) & 0xffu;
    uint32_t man = b & 0x7fffffu;
    if (exp == 0xffu) return (uint16_t)(sign | 0x7c00u | (man ? 0x200u | (man >> 13) : 0u));
    int e = (int)exp - 127 + 15;
    if (e >= 31) return (uint16_t)(sign | 0x7c00u);
    if (e <= 0) {
        if (e < -10) return (uint16_t)sign;
        uint32_t m = man | 0x800000u;
        uint32_t shift = (uint32_t)(14 - e);
        uint32_t h = m >> shift;
        uint32_t rem = m & ((1u << shift) - 1u), halfway = 1u << (shift - 1u);
        if (rem > halfway || (rem == halfway && (h & 1u))) h++;
        return (uint16_t)(sign | h);
    }
    uint32_t h = ((uint32_t)e << 10) | (man >> 13);
    uint32_t rem = man & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h++; /* may carry into inf: correct */
    return (uint16_t)(sign | h);
}

float bco_f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h >> 15) << 31;
    uint32_t exp = (h >> 10) & 0x1fu, man = h & 0x3ffu, bits;
    if (exp == 0) {
        if (man == 0) {
            bits = sign;
        } else {
            int e = -1;
            do {
                e++;
                man <<= 1;
            } while (!(man & 0x400u));
            bits = sign | ((uint32_t)(127 - 15 - e) << 23) | ((man & 0x3ffu) << 13);
        }
    } else if (exp == 31) {
        bits = sign | 0x7f800000u | (man << 13);
    } else {
        bits = sign | ((exp + 127 - 15) << 23) | (man << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

void bco_round_f16(float* x, size_t n) {
    for (size_t i = 0; i < n; i++) x[i] = bco_f16_to_f32(bco_f32_to_f16(x[i]));
}

uint64_t bco_splitmix64(uint64_t* state) {
    uint64_t z = (*state += 0x9e3779b97f4a7c15ull);
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
    return z ^ (z >> 31);
}

/* u1 in (0, 1], u2 in [0, 1) from the top 53 bits; z0 = r cos(2 pi u2), z1 = r sin(2 pi u2)
 * with r = sqrt(-2 ln u1), in double, rounded to float. */
void bco_normal(uint64_t seed, float* out, size_t n) {
    uint64_t s = seed;
    const double two_pi = 6.283185307179586476925286766559;
    for (size_t i = 0; i < n; i += 2) {
        double u1 = ((double)(bco_splitmix64(&s) >> 11) + 1.0) * 0x1.0p-53;
        double u2 = (double)(bco_splitmix64(&s) >> 11) * 0x1.0p-53;
        double r = sqrt(-2.0 * log(u1));
        out[i] = (float)(r * cos(two_pi * u2));
        if (i + 1 < n) out[i + 1] = (float)(r * sin(two_pi * u2));
    }
}
