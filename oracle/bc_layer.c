/* CPU oracle for the rest of bc-infer's layer (norms, elementwise ops, the GGUF block-format
 * product): TEST INFRASTRUCTURE, NOT PRODUCT CODE. Only tests/ and bench.py's cpu_baseline
 * leg use it, as the checker. Built with -ffp-contract=off like bc_oracle.c. Reference
 * citations are per function (paths inside the Harshil089/Borrowed-Compute checkout). */
#include "bc_oracle.h"

#include <math.h>
#include <string.h>

/* quant.rs:69-82: weights and bytes per block; 0 for an unknown type. */
int bcl_block(uint32_t ty, uint32_t* weights, uint32_t* bytes) {
    uint32_t n, b;
    switch (ty) {
        case BCL_F32: n = 1; b = 4; break;
        case BCL_F16: case BCL_BF16: n = 1; b = 2; break;
        case BCL_Q4_0: n = 32; b = 18; break;
        case BCL_Q4_1: n = 32; b = 20; break;
        case BCL_Q5_0: n = 32; b = 22; break;
        case BCL_Q5_1: n = 32; b = 24; break;
        case BCL_Q8_0: n = 32; b = 34; break;
        case BCL_Q4K: n = 256; b = 144; break;
        case BCL_Q5K: n = 256; b = 176; break;
        case BCL_Q6K: n = 256; b = 210; break;
        default: return 0;
    }
    *weights = n;
    *bytes = b;
    return 1;
}

/* quant.rs:114-131, the reference's own f32 -> f16 (round half up on the dropped bits,
 * subnormal results flushed to zero): the fixtures' scales go through it. */
uint16_t bcl_ref_f32_to_f16(float x) {
    uint32_t b;
    memcpy(&b, &x, 4);
    uint16_t sign = (uint16_t)((b >> 16) & 0x8000u);
    int32_t exp = (int32_t)((b >> 23) & 0xffu) - 127 + 15;
    uint32_t man = b & 0x7fffffu;
    if (exp >= 31) return (uint16_t)(sign | 0x7c00u);
    if (exp <= 0) return sign;
    uint32_t h = (uint32_t)sign | ((uint32_t)exp << 10) | (man >> 13);
    if (man & 0x1000u) h += 1;
    return (uint16_t)h;
}

static float f16_at(const uint8_t* b, size_t i) { return bco_f16_to_f32((uint16_t)(b[i] | (b[i + 1] << 8))); }

/* quant.rs:136-146 (ggml's get_scale_min_k4). */
void bcl_scale_min_k4(uint32_t j, const uint8_t* q, float* sc, float* mn) {
    if (j < 4) {
        *sc = (float)(q[j] & 63u);
        *mn = (float)(q[j + 4] & 63u);
    } else {
        *sc = (float)((q[j + 4] & 0xfu) | ((q[j - 4] >> 6) << 4));
        *mn = (float)((q[j + 4] >> 4) | ((q[j] >> 6) << 4));
    }
}

/* quant.rs:150-259: one block of `ty` from src into dst (block-sized). Each expression keeps
 * the reference's association (f32, every product and sum rounded on its own). */
void bcl_dequant_block(uint32_t ty, const uint8_t* src, float* dst) {
    switch (ty) {
        case BCL_F32: memcpy(dst, src, 4); break;
        case BCL_F16: dst[0] = f16_at(src, 0); break;
        case BCL_BF16: {
            uint32_t bits = (uint32_t)(src[0] | (src[1] << 8)) << 16;
            memcpy(dst, &bits, 4);
            break;
        }
        case BCL_Q4_0: {
            float d = f16_at(src, 0);
            for (int j = 0; j < 16; j++) {
                dst[j] = ((float)(src[2 + j] & 0xf) - 8.0f) * d;
                dst[j + 16] = ((float)(src[2 + j] >> 4) - 8.0f) * d;
            }
            break;
        }
        case BCL_Q4_1: {
            float d = f16_at(src, 0), m = f16_at(src, 2);
            for (int j = 0; j < 16; j++) {
                dst[j] = (float)(src[4 + j] & 0xf) * d + m;
                dst[j + 16] = (float)(src[4 + j] >> 4) * d + m;
            }
            break;
        }
        case BCL_Q5_0:
        case BCL_Q5_1: {
            const int q50 = ty == BCL_Q5_0;
            float d = f16_at(src, 0), m = q50 ? 0.0f : f16_at(src, 2);
            int at = q50 ? 2 : 4;
            uint32_t qh = (uint32_t)src[at] | ((uint32_t)src[at + 1] << 8) | ((uint32_t)src[at + 2] << 16) |
                          ((uint32_t)src[at + 3] << 24);
            const uint8_t* qs = src + at + 4;
            float offset = q50 ? 16.0f : 0.0f;
            for (int j = 0; j < 16; j++) {
                uint32_t h0 = ((qh >> j) << 4) & 0x10u;
                uint32_t h1 = (qh >> (j + 12)) & 0x10u;
                dst[j] = ((float)((qs[j] & 0xfu) | h0) - offset) * d + m;
                dst[j + 16] = ((float)((uint32_t)(qs[j] >> 4) | h1) - offset) * d + m;
            }
            break;
        }
        case BCL_Q8_0: {
            float d = f16_at(src, 0);
            for (int j = 0; j < 32; j++) dst[j] = (float)(int8_t)src[2 + j] * d;
            break;
        }
        case BCL_Q4K: {
            float d = f16_at(src, 0), dmin = f16_at(src, 2);
            const uint8_t *scales = src + 4, *qs = src + 16;
            for (int g = 0; g < 4; g++) {
                float sc1, m1, sc2, m2;
                bcl_scale_min_k4(2 * g, scales, &sc1, &m1);
                bcl_scale_min_k4(2 * g + 1, scales, &sc2, &m2);
                const uint8_t* q = qs + 32 * g;
                float* out = dst + 64 * g;
                for (int l = 0; l < 32; l++) {
                    out[l] = d * sc1 * (float)(q[l] & 0xf) - dmin * m1;
                    out[l + 32] = d * sc2 * (float)(q[l] >> 4) - dmin * m2;
                }
            }
            break;
        }
        case BCL_Q5K: {
            float d = f16_at(src, 0), dmin = f16_at(src, 2);
            const uint8_t *scales = src + 4, *qh = src + 16, *qs = src + 48;
            for (int g = 0; g < 4; g++) {
                float sc1, m1, sc2, m2;
                bcl_scale_min_k4(2 * g, scales, &sc1, &m1);
                bcl_scale_min_k4(2 * g + 1, scales, &sc2, &m2);
                uint8_t u1 = (uint8_t)(1u << (2 * g)), u2 = (uint8_t)(2u << (2 * g));
                const uint8_t* q = qs + 32 * g;
                float* out = dst + 64 * g;
                for (int l = 0; l < 32; l++) {
                    int hi1 = (qh[l] & u1) ? 16 : 0, hi2 = (qh[l] & u2) ? 16 : 0;
                    out[l] = d * sc1 * (float)((q[l] & 0xf) + hi1) - dmin * m1;
                    out[l + 32] = d * sc2 * (float)((q[l] >> 4) + hi2) - dmin * m2;
                }
            }
            break;
        }
        case BCL_Q6K: {
            const uint8_t *ql0 = src, *qh0 = src + 128, *sc0 = src + 192;
            float d = f16_at(src, 208);
            for (int half = 0; half < 2; half++) {
                const uint8_t *ql = ql0 + 64 * half, *qh = qh0 + 32 * half, *sc = sc0 + 8 * half;
                float* out = dst + 128 * half;
                for (int l = 0; l < 32; l++) {
                    int is = l / 16;
                    int q1 = (int)((ql[l] & 0xf) | ((qh[l] & 3) << 4)) - 32;
                    int q2 = (int)((ql[l + 32] & 0xf) | (((qh[l] >> 2) & 3) << 4)) - 32;
                    int q3 = (int)((ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32;
                    int q4 = (int)((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32;
                    out[l] = d * (float)(int8_t)sc[is] * (float)q1;
                    out[l + 32] = d * (float)(int8_t)sc[is + 2] * (float)q2;
                    out[l + 64] = d * (float)(int8_t)sc[is + 4] * (float)q3;
                    out[l + 96] = d * (float)(int8_t)sc[is + 6] * (float)q4;
                }
            }
            break;
        }
        default: break;
    }
}

/* quant.rs:349-355 per row: rows x cols weights of `ty` (rows of whole blocks) to f32. */
int bcl_dequant(uint32_t ty, const uint8_t* data, uint64_t rows, uint64_t cols, float* out) {
    uint32_t n, b;
    if (!bcl_block(ty, &n, &b) || cols % n) return -1;
    const uint64_t row_bytes = cols / n * b;
    for (uint64_t r = 0; r < rows; r++)
        for (uint64_t k = 0; k < cols / n; k++) bcl_dequant_block(ty, data + r * row_bytes + k * b, out + r * cols + k * n);
    return 0;
}

static uint64_t xorshift(uint64_t* s) {
    *s ^= *s << 13;
    *s ^= *s >> 7;
    *s ^= *s << 17;
    return *s;
}

/* fixtures.rs:66-92 (random_tensor): the bytes of a rows x cols tensor of `ty`, random
 * weights and modest scales, from a seeded xorshift64 (13, 7, 17): every byte first, then
 * each block's scale fields (or whole value, for the plain types) rewritten in order. */
int bcl_random_tensor(uint32_t ty, uint64_t rows, uint64_t cols, uint64_t seed, uint8_t* out) {
    uint32_t n, size;
    if (!bcl_block(ty, &n, &size) || (rows * cols) % n) return -1;
    uint64_t s = seed * 0x9e3779b97f4a7c15ull | 1u;
    const uint64_t len = rows * cols / n * size;
    for (uint64_t i = 0; i < len; i++) out[i] = (uint8_t)xorshift(&s);
    for (uint64_t at = 0; at < len; at += size) {
        uint8_t* blk = out + at;
        if (ty == BCL_F32) {
            float v = ((float)(xorshift(&s) % 2001) - 1000.0f) / 1000.0f;
            memcpy(blk, &v, 4);
        } else if (ty == BCL_F16) {
            uint16_t h = bcl_ref_f32_to_f16(((float)(xorshift(&s) % 2001) - 1000.0f) / 1000.0f);
            memcpy(blk, &h, 2);
        } else if (ty == BCL_BF16) {
            float v = ((float)(xorshift(&s) % 2001) - 1000.0f) / 1000.0f;
            uint32_t bits;
            memcpy(&bits, &v, 4);
            uint16_t h = (uint16_t)(bits >> 16);
            memcpy(blk, &h, 2);
        } else {
            const int f = ty == BCL_Q6K ? 208 : 0;
            uint16_t h = bcl_ref_f32_to_f16(((float)(xorshift(&s) % 1000) + 1.0f) / 40000.0f);
            memcpy(blk + f, &h, 2);
            if (ty == BCL_Q4_1 || ty == BCL_Q5_1 || ty == BCL_Q4K || ty == BCL_Q5K) {
                h = bcl_ref_f32_to_f16(((float)(xorshift(&s) % 1000) + 1.0f) / 40000.0f);
                memcpy(blk + 2, &h, 2);
            }
        }
    }
    return 0;
}

/* quant.rs:634-646: f32 weights (a whole number of 32-blocks) to Q8_0 (34 bytes a block). */
void bcl_quantize_q8_0(const float* v, uint64_t n, uint8_t* out) {
    for (uint64_t b = 0; b < n / 32; b++) {
        const float* x = v + 32 * b;
        uint8_t* o = out + 34 * b;
        float mx = 0.0f;
        for (int i = 0; i < 32; i++) mx = fmaxf(mx, fabsf(x[i]));
        float d = mx / 127.0f;
        float inv = d > 0.0f ? 1.0f / d : 0.0f;
        uint16_t h = bcl_ref_f32_to_f16(d);
        memcpy(o, &h, 2);
        for (int i = 0; i < 32; i++) {
            float q = roundf(x[i] * inv); /* Rust's round: half away from zero, as roundf */
            q = q < -127.0f ? -127.0f : (q > 127.0f ? 127.0f : q);
            o[2 + i] = (uint8_t)(int8_t)q;
        }
    }
}

/* gpu/mod.rs:193-196 (Gpu::self_check's reference): out[i][r] = sum_c W[r][c] x[i][c] in
 * f64 over the dequantized weights, for the first `rows` weight rows. */
int bcl_matmul_f64(uint32_t ty, const uint8_t* data, uint64_t rows, uint64_t cols, const float* x, uint64_t n,
                   double* out) {
    uint32_t bn, bb;
    if (!bcl_block(ty, &bn, &bb) || cols % bn) return -1;
    const uint64_t row_bytes = cols / bn * bb;
    float w[256];
    for (uint64_t r = 0; r < rows; r++) {
        for (uint64_t i = 0; i < n; i++) out[i * rows + r] = 0.0;
        for (uint64_t k = 0; k < cols / bn; k++) {
            bcl_dequant_block(ty, data + r * row_bytes + k * bb, w);
            for (uint64_t i = 0; i < n; i++) {
                double acc = out[i * rows + r];
                for (uint32_t j = 0; j < bn; j++) acc += (double)w[j] * (double)x[i * cols + k * bn + j];
                out[i * rows + r] = acc;
            }
        }
    }
    return 0;
}

/* model.rs:381-388: per row, scale = 1 / sqrt(dot(row, row) / len + eps) (quant.rs:617-631's
 * dot), out = v * scale * w, each product rounded. */
void bcl_rms_norm(const float* x, const float* w, float* out, uint64_t rows, uint64_t cols, float eps) {
    for (uint64_t r = 0; r < rows; r++) {
        const float* row = x + r * cols;
        float ms = bco_dot(row, row, cols) / (float)cols;
        float scale = 1.0f / sqrtf(ms + eps);
        for (uint64_t c = 0; c < cols; c++) out[r * cols + c] = row[c] * scale * w[c];
    }
}

/* model.rs:343: g <- g / (1 + exp(-g)) * u. */
void bcl_silu_mul(float* g, const float* u, uint64_t n) {
    for (uint64_t i = 0; i < n; i++) g[i] = g[i] / (1.0f + expf(-g[i])) * u[i];
}

/* model.rs:371-377 (add_bias): each dim-long row of x plus b. */
void bcl_bias_add(float* x, const float* b, uint64_t n, uint64_t dim) {
    for (uint64_t i = 0; i < n; i++) x[i] += b[i % dim];
}

/* model.rs:337, 345: x += y. */
void bcl_add(float* x, const float* y, uint64_t n) {
    for (uint64_t i = 0; i < n; i++) x[i] += y[i];
}
