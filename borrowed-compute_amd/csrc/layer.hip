// The rest of bc-infer's layer on the GPU: the GGUF block-format matrix product
// (crates/bc-infer/src/gpu/kernels.h:51-214, entry cuda.cu:77-79), RMSNorm (kernels.h:216-225,
// cuda.cu:80) and the elementwise ops (kernels.h:327-330, cuda.cu:86-88).
//
// Product layout: weights stay in their ggml blocks, rows of whole blocks (row_bytes =
// cols / block_weights * block_bytes); every format is read a "group" of 32 weights at a
// time. A wave owns ROWS_PER_WAVE weight rows and its 64 lanes take groups l, l + 64, ...
// of them: per group the lane loads its input values once (up to NB input rows) and
// dequantizes each of its rows' 32 weights once, with quant.rs's per-weight expression, then
// sums weight x input in a fixed order. The 64 lane sums meet in a fixed butterfly. So an
// input row's result depends on that row alone, never on how many rows share the batch,
// and reruns give the same bits (the reference kernel's properties, kernels.h:9-11).
#include "common.hpp"
#include "internal.hpp"

namespace bchip {

// ggml type numbers (quant.rs:35-49).
enum : uint32_t {
    G_F32 = 0, G_F16 = 1, G_Q4_0 = 2, G_Q4_1 = 3, G_Q5_0 = 6, G_Q5_1 = 7, G_Q8_0 = 8,
    G_Q4K = 12, G_Q5K = 13, G_Q6K = 14, G_BF16 = 30,
};

bool ggml_block(uint32_t ty, uint32_t& weights, uint32_t& bytes) {
    switch (ty) {
        case G_F32: weights = 1; bytes = 4; return true;
        case G_F16: case G_BF16: weights = 1; bytes = 2; return true;
        case G_Q4_0: weights = 32; bytes = 18; return true;
        case G_Q4_1: weights = 32; bytes = 20; return true;
        case G_Q5_0: weights = 32; bytes = 22; return true;
        case G_Q5_1: weights = 32; bytes = 24; return true;
        case G_Q8_0: weights = 32; bytes = 34; return true;
        case G_Q4K: weights = 256; bytes = 144; return true;
        case G_Q5K: weights = 256; bytes = 176; return true;
        case G_Q6K: weights = 256; bytes = 210; return true;
        default: return false;
    }
}

constexpr int NB = 8;             // input rows a pass (grid.y) takes
constexpr int ROWS_PER_WAVE = 4;  // weight rows a wave owns
constexpr int MM_WAVES = 4;       // waves a workgroup

__device__ __forceinline__ float h2f(uint32_t bits16) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)bits16);
}
__device__ __forceinline__ uint32_t ld16(const uint8_t* p) { return *(const uint16_t*)p; }
// Four bytes at a 2-byte-aligned address.
__device__ __forceinline__ uint32_t ld32h(const uint8_t* p) { return ld16(p) | (ld16(p + 2) << 16); }
__device__ __forceinline__ uint32_t ld32(const uint8_t* p) { return *(const uint32_t*)p; }
__device__ __forceinline__ float i8f(uint32_t b) { return (float)(int8_t)(uint8_t)b; }

// quant.rs:136-146.
__device__ __forceinline__ void scale_min_k4(uint32_t j, const uint8_t* q, float& sc, float& mn) {
    if (j < 4) {
        sc = (float)(q[j] & 63u);
        mn = (float)(q[j + 4] & 63u);
    } else {
        sc = (float)((q[j + 4] & 15u) | ((q[j - 4] >> 6) << 4));
        mn = (float)((q[j + 4] >> 4) | ((q[j] >> 6) << 4));
    }
}

// The 32 weights of group g of a stored row, w[j] = weight 32g + j, each by its format's
// expression in quant.rs:150-259 (same association, so each weight has the bits the CPU's
// dequantization gives it).
template <uint32_t TY>
__device__ __forceinline__ void group_weights(const uint8_t* __restrict__ row, uint32_t g, float (&w)[32]) {
    if constexpr (TY == G_F32) {
        const float4* p = (const float4*)(row + (size_t)g * 128);
#pragma unroll
        for (int k = 0; k < 8; k++) {
            const float4 v = p[k];
            w[4 * k] = v.x; w[4 * k + 1] = v.y; w[4 * k + 2] = v.z; w[4 * k + 3] = v.w;
        }
    } else if constexpr (TY == G_F16 || TY == G_BF16) {
        const uint4* p = (const uint4*)(row + (size_t)g * 64);
#pragma unroll
        for (int k = 0; k < 4; k++) {
            const uint4 v = p[k];
            const uint32_t u[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
            for (int j = 0; j < 4; j++) {
                if constexpr (TY == G_F16) {
                    w[8 * k + 2 * j] = h2f(u[j] & 0xffffu);
                    w[8 * k + 2 * j + 1] = h2f(u[j] >> 16);
                } else {
                    w[8 * k + 2 * j] = __uint_as_float(u[j] << 16);
                    w[8 * k + 2 * j + 1] = __uint_as_float(u[j] & 0xffff0000u);
                }
            }
        }
    } else if constexpr (TY == G_Q4_0 || TY == G_Q5_0 || TY == G_Q8_0) {
        // 2-byte-aligned blocks: 16-bit loads.
        const uint8_t* b = row + (size_t)g * (TY == G_Q4_0 ? 18 : TY == G_Q5_0 ? 22 : 34);
        const float d = h2f(ld16(b));
        if constexpr (TY == G_Q8_0) {
#pragma unroll
            for (int k = 0; k < 8; k++) {
                const uint32_t v = ld32h(b + 2 + 4 * k);
#pragma unroll
                for (int j = 0; j < 4; j++) w[4 * k + j] = i8f(v >> (8 * j)) * d;
            }
        } else {
            const uint8_t* qs = b + (TY == G_Q4_0 ? 2 : 6);
            const uint32_t qh = TY == G_Q5_0 ? ld32h(b + 2) : 0u;
            const float off = TY == G_Q4_0 ? 8.0f : 16.0f;
#pragma unroll
            for (int k = 0; k < 4; k++) {
                const uint32_t v = ld32h(qs + 4 * k);
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    const uint32_t e = 4 * k + j, byte = (v >> (8 * j)) & 255u;
                    uint32_t lo = byte & 15u, hi = byte >> 4;
                    if constexpr (TY == G_Q5_0) {
                        lo |= ((qh >> e) << 4) & 16u;
                        hi |= (qh >> (e + 12)) & 16u;
                    }
                    // Q5_0 adds its zero minimum as quant.rs does (-0 becomes +0).
                    w[e] = TY == G_Q5_0 ? ((float)lo - off) * d + 0.0f : ((float)lo - off) * d;
                    w[e + 16] = TY == G_Q5_0 ? ((float)hi - off) * d + 0.0f : ((float)hi - off) * d;
                }
            }
        }
    } else if constexpr (TY == G_Q4_1 || TY == G_Q5_1) {
        const uint8_t* b = row + (size_t)g * (TY == G_Q4_1 ? 20 : 24);
        const uint32_t dm = ld32(b);
        const float d = h2f(dm & 0xffffu), m = h2f(dm >> 16);
        const uint8_t* qs = b + (TY == G_Q4_1 ? 4 : 8);
        const uint32_t qh = TY == G_Q5_1 ? ld32(b + 4) : 0u;
#pragma unroll
        for (int k = 0; k < 4; k++) {
            const uint32_t v = ld32(qs + 4 * k);
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const uint32_t e = 4 * k + j, byte = (v >> (8 * j)) & 255u;
                uint32_t lo = byte & 15u, hi = byte >> 4;
                if constexpr (TY == G_Q5_1) {
                    lo |= ((qh >> e) << 4) & 16u;
                    hi |= (qh >> (e + 12)) & 16u;
                }
                w[e] = (float)lo * d + m;
                w[e + 16] = (float)hi * d + m;
            }
        }
    } else if constexpr (TY == G_Q4K || TY == G_Q5K) {
        // 256 weights a block in 4 chunks of 64: group 2c is chunk c's low nibbles, 2c + 1 its
        // high nibbles.
        const uint8_t* b = row + (size_t)(g / 8) * (TY == G_Q4K ? 144 : 176);
        const uint32_t sub = g % 8, c = sub / 2, hi = sub % 2;
        const uint32_t dd = ld32(b);
        const float d = h2f(dd & 0xffffu), dmin = h2f(dd >> 16);
        float sc, mn;
        scale_min_k4(sub, b + 4, sc, mn);
        const float ds = d * sc, dm = dmin * mn;
        const uint8_t* qs = b + (TY == G_Q4K ? 16 : 48) + 32 * c;
#pragma unroll
        for (int k = 0; k < 8; k++) {
            const uint32_t v = ld32(qs + 4 * k);
            const uint32_t h = TY == G_Q5K ? ld32(b + 16 + 4 * k) : 0u;
#pragma unroll
            for (int j = 0; j < 4; j++) {
                uint32_t q = (v >> (8 * j + 4 * hi)) & 15u;
                if constexpr (TY == G_Q5K) q += ((h >> (8 * j + 2 * c + hi)) & 1u) << 4;
                w[4 * k + j] = ds * (float)q - dm;
            }
        }
    } else if constexpr (TY == G_Q6K) {
        // Half hh, quarter qr of a 256-block: ql bytes 64hh + 32(qr % 2) .., nibble qr / 2;
        // qh bytes 128 + 32hh .., bits 2qr; scales 192 + 8hh + 2qr (+1 for weights 16..31).
        const uint8_t* b = row + (size_t)(g / 8) * 210;
        const uint32_t sub = g % 8, hh = sub / 4, qr = sub % 4;
        const uint8_t* ql = b + 64 * hh + ((qr & 1u) ? 32 : 0);
        const uint8_t* qh = b + 128 + 32 * hh;
        const float d = h2f(ld16(b + 208));
        const uint32_t scs = ld16(b + 192 + 8 * hh + 2 * qr);
        const float d0 = d * i8f(scs & 255u), d1 = d * i8f(scs >> 8);
        const uint32_t shift = qr < 2 ? 0 : 4;
#pragma unroll
        for (int k = 0; k < 8; k++) {
            const uint32_t lo = ld32h(ql + 4 * k), h = ld32h(qh + 4 * k);
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const int q = (int)(((lo >> (8 * j + shift)) & 15u) | (((h >> (8 * j + 2 * qr)) & 3u) << 4)) - 32;
                w[4 * k + j] = (k < 4 ? d0 : d1) * (float)q;
            }
        }
    }
}

// Sum over a wave of one value per lane, the same butterfly for every call.
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m, 64);
    return v;
}

struct MatmulParams {
    const uint8_t* w;
    const float* x;
    float* out;
    uint32_t rows, cols, n, row_bytes;
};

// out[i][r] = sum_c W[r][c] x[i][c]: workgroup (blockIdx.x) = MM_WAVES waves x ROWS_PER_WAVE
// weight rows, blockIdx.y = input rows i0 .. i0 + NB.
template <uint32_t TY>
__global__ __launch_bounds__(64 * MM_WAVES) void k_matmul(const MatmulParams p) {
    const uint32_t lane = threadIdx.x & 63;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t r0 = (blockIdx.x * MM_WAVES + wave) * ROWS_PER_WAVE;
    if (r0 >= p.rows) return;
    const uint32_t i0 = blockIdx.y * NB;
    const uint32_t nb = min((uint32_t)NB, p.n - i0);
    const uint32_t groups = p.cols / 32;
    float acc[NB][ROWS_PER_WAVE];
#pragma unroll
    for (int i = 0; i < NB; i++)
#pragma unroll
        for (int r = 0; r < ROWS_PER_WAVE; r++) acc[i][r] = 0.0f;
    // Rows past the matrix read row r0 again (their sums are never stored).
    const uint8_t* rowp[ROWS_PER_WAVE];
#pragma unroll
    for (int r = 0; r < ROWS_PER_WAVE; r++)
        rowp[r] = p.w + (size_t)(r0 + r < p.rows ? r0 + r : r0) * p.row_bytes;
    for (uint32_t g = lane; g < groups; g += 64) {
        float w[ROWS_PER_WAVE][32];
#pragma unroll
        for (int r = 0; r < ROWS_PER_WAVE; r++) group_weights<TY>(rowp[r], g, w[r]);
#pragma unroll
        for (int i = 0; i < NB; i++) {
            if (i < (int)nb) {
                const float4* xg = (const float4*)(p.x + (size_t)(i0 + i) * p.cols + 32 * g);
                float xv[32];
#pragma unroll
                for (int k = 0; k < 8; k++) {
                    const float4 v = xg[k];
                    xv[4 * k] = v.x; xv[4 * k + 1] = v.y; xv[4 * k + 2] = v.z; xv[4 * k + 3] = v.w;
                }
#pragma unroll
                for (int r = 0; r < ROWS_PER_WAVE; r++) {
                    float s = 0.0f;
#pragma unroll
                    for (int j = 0; j < 32; j++) s += w[r][j] * xv[j];
                    acc[i][r] += s;
                }
            }
        }
    }
#pragma unroll
    for (int i = 0; i < NB; i++) {
        if (i < (int)nb) {
#pragma unroll
            for (int r = 0; r < ROWS_PER_WAVE; r++) {
                const float s = wave_sum(acc[i][r]);
                if (lane == 0 && r0 + r < p.rows) p.out[(size_t)(i0 + i) * p.rows + r0 + r] = s;
            }
        }
    }
}

template <uint32_t TY>
static hipError_t matmul_t(const MatmulParams& mp, hipStream_t s) {
    const uint32_t per_wg = MM_WAVES * ROWS_PER_WAVE;
    const dim3 grid((mp.rows + per_wg - 1) / per_wg, (mp.n + NB - 1) / NB);
    hipLaunchKernelGGL((k_matmul<TY>), grid, dim3(64 * MM_WAVES), 0, s, mp);
    return hipGetLastError();
}

hipError_t matmul_launch(const void* w, uint32_t type, const float* x, float* out, uint32_t rows, uint32_t cols,
                         uint32_t n, uint32_t row_bytes, hipStream_t s) {
    const MatmulParams mp{(const uint8_t*)w, x, out, rows, cols, n, row_bytes};
    switch (type) {
        case G_F32: return matmul_t<G_F32>(mp, s);
        case G_F16: return matmul_t<G_F16>(mp, s);
        case G_BF16: return matmul_t<G_BF16>(mp, s);
        case G_Q4_0: return matmul_t<G_Q4_0>(mp, s);
        case G_Q4_1: return matmul_t<G_Q4_1>(mp, s);
        case G_Q5_0: return matmul_t<G_Q5_0>(mp, s);
        case G_Q5_1: return matmul_t<G_Q5_1>(mp, s);
        case G_Q8_0: return matmul_t<G_Q8_0>(mp, s);
        case G_Q4K: return matmul_t<G_Q4K>(mp, s);
        case G_Q5K: return matmul_t<G_Q5K>(mp, s);
        case G_Q6K: return matmul_t<G_Q6K>(mp, s);
        default: return hipErrorInvalidValue;
    }
}

// RMSNorm, one workgroup a row: the sum of squares over the workgroup's threads (4 values
// each step, a fixed tree), scale = 1 / sqrt(mean + eps), out = x * scale * w.
constexpr int NORM_THREADS = 256;

// vec: cols % 4 == 0 and every pointer 16-byte aligned (float4 accesses).
__global__ __launch_bounds__(NORM_THREADS) void k_rms_norm(const float* __restrict__ x, const float* __restrict__ w,
                                                           float* __restrict__ out, uint32_t cols, float eps,
                                                           bool vec) {
    __shared__ float part[NORM_THREADS / 64];
    const float* xr = x + (size_t)blockIdx.x * cols;
    float* orow = out + (size_t)blockIdx.x * cols;
    const uint32_t t = threadIdx.x;
    float s = 0.0f;
    if (vec) {
        for (uint32_t c = 4 * t; c < cols; c += 4 * NORM_THREADS) {
            const float4 v = *(const float4*)(xr + c);
            s += v.x * v.x + v.y * v.y + v.z * v.z + v.w * v.w;
        }
    } else {
        for (uint32_t c = t; c < cols; c += NORM_THREADS) s += xr[c] * xr[c];
    }
    s = wave_sum(s);
    if ((t & 63) == 0) part[t >> 6] = s;
    __syncthreads();
    float tot = 0.0f;
#pragma unroll
    for (int i = 0; i < NORM_THREADS / 64; i++) tot += part[i];
    const float scale = 1.0f / __builtin_sqrtf(tot / (float)cols + eps);
    if (vec) {
        for (uint32_t c = 4 * t; c < cols; c += 4 * NORM_THREADS) {
            const float4 v = *(const float4*)(xr + c), g = *(const float4*)(w + c);
            *(float4*)(orow + c) = float4{v.x * scale * g.x, v.y * scale * g.y, v.z * scale * g.z, v.w * scale * g.w};
        }
    } else {
        for (uint32_t c = t; c < cols; c += NORM_THREADS) orow[c] = xr[c] * scale * w[c];
    }
}

hipError_t rms_norm_launch(const float* x, const float* w, float* out, uint32_t rows, uint32_t cols, float eps,
                           bool vec, hipStream_t s) {
    hipLaunchKernelGGL(k_rms_norm, dim3(rows), dim3(NORM_THREADS), 0, s, x, w, out, cols, eps, vec);
    return hipGetLastError();
}

// Elementwise ops, grid-stride. silu's e^-v is 2^(-v log2 e) on the hardware's exp2, as the
// reference kernels compute it (cuda.cu:66).

template <int OP>
__global__ __launch_bounds__(256) void k_elementwise(float* __restrict__ x, const float* __restrict__ y, uint64_t n,
                                                     uint32_t dim) {
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (uint64_t)gridDim.x * blockDim.x) {
        if constexpr (OP == EW_BIAS) {
            x[i] += y[i % dim];
        } else if constexpr (OP == EW_SILU_MUL) {
            const float v = x[i];
            x[i] = v / (1.0f + __builtin_amdgcn_exp2f(-v * LOG2E)) * y[i];
        } else {
            x[i] += y[i];
        }
    }
}

hipError_t elementwise_launch(int op, float* x, const float* y, uint64_t n, uint32_t dim, hipStream_t s) {
    const uint64_t blocks64 = (n + 255) / 256;
    const uint32_t blocks = (uint32_t)(blocks64 < 8192 ? blocks64 : 8192);
    switch (op) {
        case EW_BIAS: hipLaunchKernelGGL(k_elementwise<EW_BIAS>, dim3(blocks), dim3(256), 0, s, x, y, n, dim); break;
        case EW_SILU_MUL:
            hipLaunchKernelGGL(k_elementwise<EW_SILU_MUL>, dim3(blocks), dim3(256), 0, s, x, y, n, dim);
            break;
        default: hipLaunchKernelGGL(k_elementwise<EW_ADD>, dim3(blocks), dim3(256), 0, s, x, y, n, dim); break;
    }
    return hipGetLastError();
}

}  // namespace bchip
