// The rest of bc-infer's layer on the GPU: the GGUF block-format matrix product
// (crates/bc-infer/src/gpu/kernels.h:51-214, entry cuda.cu:77-79), RMSNorm (kernels.h:216-225,
// cuda.cu:80) and the elementwise ops (kernels.h:327-330, cuda.cu:86-88).
//
// Product layout: weights stay in their ggml blocks, rows of whole blocks (row_bytes =
// cols / block_weights * block_bytes); every format is read a "group" of 32 weights at a
// time. A wave owns R weight rows and its 64 lanes take the row's groups, one each per
// column tile: per group the lane loads its rows' packed bytes and its input values (up to
// NB input rows), unpacks each row's 32 quants and sums in a fixed order. The 64 lane sums meet in a
// fixed butterfly. So an input row's result depends on that row alone, never on how many
// rows share the batch, and reruns give the same bits (the reference kernel's properties,
// kernels.h:9-11).
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

constexpr int NB = 8;  // input rows a pass (grid.y) takes

__device__ __forceinline__ float h2f(uint32_t bits16) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)bits16);
}
__device__ __forceinline__ uint32_t ld16(const uint8_t* p) { return *(const uint16_t*)p; }
// Four bytes at a 2-byte-aligned address.
__device__ __forceinline__ uint32_t ld32h(const uint8_t* p) { return ld16(p) | (ld16(p + 2) << 16); }
__device__ __forceinline__ uint32_t ld32(const uint8_t* p) { return *(const uint32_t*)p; }
__device__ __forceinline__ float i8f(uint32_t b) { return (float)(int8_t)(uint8_t)b; }

// A group's bytes are loaded first (packed, PK<TY> dwords: a few registers a group, so a
// wave can hold several rows' groups in flight) and unpacked just before use.
template <uint32_t TY>
constexpr int PK = TY == G_F32 ? 32 : (TY == G_F16 || TY == G_BF16) ? 16 : (TY == G_Q4_0 || TY == G_Q4_1) ? 5
                 : (TY == G_Q5_0 || TY == G_Q5_1) ? 6 : TY == G_Q8_0 ? 9 : TY == G_Q4K ? 12 : TY == G_Q5K ? 20 : 17;

template <uint32_t TY>
__device__ __forceinline__ void group_load(const uint8_t* __restrict__ row, uint32_t g, uint32_t (&pk)[PK<TY>]) {
    if constexpr (TY == G_F32 || TY == G_F16 || TY == G_BF16) {
        const uint4* p = (const uint4*)(row + (size_t)g * (TY == G_F32 ? 128 : 64));
#pragma unroll
        for (int k = 0; k < PK<TY> / 4; k++) {
            const uint4 v = p[k];
            pk[4 * k] = v.x; pk[4 * k + 1] = v.y; pk[4 * k + 2] = v.z; pk[4 * k + 3] = v.w;
        }
    } else if constexpr (TY == G_Q8_0) {
        const uint8_t* b8 = row + (size_t)g * 34;
        pk[0] = ld16(b8);
#pragma unroll
        for (int k = 0; k < 8; k++) pk[1 + k] = ld32h(b8 + 2 + 4 * k);
    } else if constexpr (TY == G_Q4_0 || TY == G_Q5_0 || TY == G_Q4_1 || TY == G_Q5_1) {
        constexpr bool Q41 = TY == G_Q4_1 || TY == G_Q5_1, FIVE = TY == G_Q5_0 || TY == G_Q5_1;
        constexpr uint32_t BS = TY == G_Q4_0 ? 18 : TY == G_Q4_1 ? 20 : TY == G_Q5_0 ? 22 : 24;
        const uint8_t* bb = row + (size_t)g * BS;
        pk[0] = Q41 ? ld32(bb) : ld16(bb);  // d (and m)
        if constexpr (FIVE) pk[5] = ld32h(bb + (Q41 ? 4 : 2));
        const uint8_t* qs = bb + (Q41 ? 4 : 2) + (FIVE ? 4 : 0);
#pragma unroll
        for (int k = 0; k < 4; k++) pk[1 + k] = Q41 ? ld32(qs + 4 * k) : ld32h(qs + 4 * k);
    } else if constexpr (TY == G_Q4K || TY == G_Q5K) {
        const uint8_t* bb = row + (size_t)(g / 8) * (TY == G_Q4K ? 144 : 176);
        const uint32_t c = (g % 8) / 2;
#pragma unroll
        for (int k = 0; k < 4; k++) pk[k] = ld32(bb + 4 * k);  // d, dmin, the 12 scale bytes
        const uint8_t* qs = bb + (TY == G_Q4K ? 16 : 48) + 32 * c;
#pragma unroll
        for (int k = 0; k < 8; k++) pk[4 + k] = ld32(qs + 4 * k);
        if constexpr (TY == G_Q5K) {
#pragma unroll
            for (int k = 0; k < 8; k++) pk[12 + k] = ld32(bb + 16 + 4 * k);
        }
    } else {  // Q6K
        const uint8_t* bb = row + (size_t)(g / 8) * 210;
        const uint32_t sub = g % 8, hh = sub / 4, qr = sub % 4;
        const uint8_t* ql = bb + 64 * hh + ((qr & 1u) ? 32 : 0);
        const uint8_t* qh = bb + 128 + 32 * hh;
#pragma unroll
        for (int k = 0; k < 8; k++) {
            pk[k] = ld32h(ql + 4 * k);
            pk[8 + k] = ld32h(qh + 4 * k);
        }
        pk[16] = ld16(bb + 192 + 8 * hh + 2 * qr) | (ld16(bb + 208) << 16);
    }
}

// Group g's quants and per-half affine maps from its packed bytes: weight j = a[h] * q[j] +
// b[h] for h = j / 16 (quant.rs:150-259's values: Q4_0 (q - 8) d, Q4_1 q d + m, Q5_0
// (q - 16) d, Q5_1 q d + m, Q8_0 q d, Q4K/Q5K ds q - dm, Q6K d_h (q - 32); the plain types
// are their values with a = 1, b = 0). The product then needs per half only sum(q x) and
// sum(x): one conversion and one FMA a weight, not a dequantization and a product.
template <uint32_t TY>
constexpr bool plain_type() {
    return TY == G_F32 || TY == G_F16 || TY == G_BF16;
}

// Bytes 0..3 of v as floats (the hardware's byte-to-float conversions).
__device__ __forceinline__ void bytes4(uint32_t v, float* q) {
    q[0] = (float)(v & 255u);
    q[1] = (float)((v >> 8) & 255u);
    q[2] = (float)((v >> 16) & 255u);
    q[3] = (float)(v >> 24);
}

template <uint32_t TY>
__device__ __forceinline__ void group_unpack(const uint32_t (&pk)[PK<TY>], uint32_t g, float (&q)[32], float (&a)[2],
                                             float (&b)[2]) {
    if constexpr (TY == G_F32) {
#pragma unroll
        for (int j = 0; j < 32; j++) q[j] = __uint_as_float(pk[j]);
    } else if constexpr (TY == G_F16 || TY == G_BF16) {
#pragma unroll
        for (int j = 0; j < 16; j++) {
            if constexpr (TY == G_F16) {
                q[2 * j] = h2f(pk[j] & 0xffffu);
                q[2 * j + 1] = h2f(pk[j] >> 16);
            } else {
                q[2 * j] = __uint_as_float(pk[j] << 16);
                q[2 * j + 1] = __uint_as_float(pk[j] & 0xffff0000u);
            }
        }
    } else if constexpr (TY == G_Q8_0) {
#pragma unroll
        for (int k = 0; k < 8; k++)
#pragma unroll
            for (int j = 0; j < 4; j++) q[4 * k + j] = i8f(pk[1 + k] >> (8 * j));
        a[0] = a[1] = h2f(pk[0]);
        b[0] = b[1] = 0.0f;
    } else if constexpr (TY == G_Q4_0 || TY == G_Q5_0 || TY == G_Q4_1 || TY == G_Q5_1) {
        // element j in byte j's low nibble, j + 16 in its high nibble; Q5 adds bit j of qh as
        // bit 4 of element j
        constexpr bool Q41 = TY == G_Q4_1 || TY == G_Q5_1, FIVE = TY == G_Q5_0 || TY == G_Q5_1;
        const float d = h2f(pk[0] & 0xffffu);
        const float m = Q41 ? h2f(pk[0] >> 16) : 0.0f;
#pragma unroll
        for (int k = 0; k < 4; k++) {
            uint32_t lo = pk[1 + k] & 0x0f0f0f0fu, hi = (pk[1 + k] >> 4) & 0x0f0f0f0fu;
            if constexpr (FIVE) {
                // bits 4k .. 4k+3 of qh to bit 4 of bytes 0..3; bits 16 + 4k .. likewise
                const uint32_t qh = pk[5];
                const uint32_t l4 = (qh >> (4 * k)) & 15u, h4 = (qh >> (16 + 4 * k)) & 15u;
                lo |= ((l4 & 1u) << 4) | ((l4 & 2u) << 11) | ((l4 & 4u) << 18) | ((l4 & 8u) << 25);
                hi |= ((h4 & 1u) << 4) | ((h4 & 2u) << 11) | ((h4 & 4u) << 18) | ((h4 & 8u) << 25);
            }
            bytes4(lo, &q[4 * k]);
            bytes4(hi, &q[16 + 4 * k]);
        }
        a[0] = a[1] = d;
        b[0] = b[1] = Q41 ? m : (TY == G_Q4_0 ? -8.0f : -16.0f) * d;
    } else if constexpr (TY == G_Q4K || TY == G_Q5K) {
        // 256 weights a block in 4 chunks of 64: group 2c is chunk c's low nibbles, 2c + 1 its
        // high nibbles (Q5K: plus bit 2c + hi of each qh byte, as bit 4).
        const uint32_t sub = g % 8, c = sub / 2, hi = sub % 2;
        const float d = h2f(pk[0] & 0xffffu), dmin = h2f(pk[0] >> 16);
        auto sbyte = [&](uint32_t k) { return (pk[1 + k / 4] >> (8 * (k % 4))) & 255u; };  // scales[k]
        float sc, mn;
        if (sub < 4) {  // quant.rs:136-146
            sc = (float)(sbyte(sub) & 63u);
            mn = (float)(sbyte(sub + 4) & 63u);
        } else {
            sc = (float)((sbyte(sub + 4) & 15u) | ((sbyte(sub - 4) >> 6) << 4));
            mn = (float)((sbyte(sub + 4) >> 4) | ((sbyte(sub) >> 6) << 4));
        }
#pragma unroll
        for (int k = 0; k < 8; k++) {
            uint32_t v = (pk[4 + k] >> (4 * hi)) & 0x0f0f0f0fu;
            if constexpr (TY == G_Q5K) v |= ((pk[12 + k] >> (2 * c + hi)) & 0x01010101u) << 4;
            bytes4(v, &q[4 * k]);
        }
        a[0] = a[1] = d * sc;
        b[0] = b[1] = -(dmin * mn);
    } else {  // Q6K: ql nibble qr / 2, qh bits 2qr, scales for weights 0..15 and 16..31
        const uint32_t qr = (g % 8) % 4, shift = qr < 2 ? 0 : 4;
#pragma unroll
        for (int k = 0; k < 8; k++) {
            const uint32_t v = ((pk[k] >> shift) & 0x0f0f0f0fu) | (((pk[8 + k] >> (2 * qr)) & 0x03030303u) << 4);
            bytes4(v, &q[4 * k]);
        }
        const float d = h2f(pk[16] >> 16);
        a[0] = d * i8f(pk[16] & 255u);
        a[1] = d * i8f((pk[16] >> 8) & 255u);
        b[0] = -32.0f * a[0];
        b[1] = -32.0f * a[1];
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

// out[i][r] = sum_c W[r][c] x[i][c]: workgroup (blockIdx.x) = MM_WAVES waves x R weight rows,
// blockIdx.y = input rows i0 .. i0 + NBT. The input rows pass through LDS in column tiles of
// 64 groups (one group a lane), read from HBM once per workgroup with coalesced loads and
// stored with a padded group stride (XS floats) so that each lane's 16-byte reads of its
// group fall on distinct banks; each lane's packed weights for the tile are loaded before
// the tile, so the two latencies overlap. Per lane, group and input row: the two half sums
// of q x (FMA chains, weights in order) and of x, then acc += a0 sq0 + a1 sq1 + b0 sx0 +
// b1 sx1 (in that order, as FMAs); the 64 lane sums meet in a fixed butterfly. R only sets
// which rows a wave holds, not a row's arithmetic.
constexpr int XS = 36;           // LDS floats per group of 32 inputs
constexpr int TILE_GROUPS = 64;  // groups per column tile: one per lane
constexpr int MM_WAVES = 4;      // waves a workgroup

template <uint32_t TY, int NBT, int R>
__global__ __launch_bounds__(64 * MM_WAVES) void k_matmul(const MatmulParams p) {
    // nb tiles of TILE_GROUPS * XS floats (dynamic: a one-row pass takes 9 KB, so more
    // workgroups share a CU).
    extern __shared__ __attribute__((aligned(16))) float xs_dyn[];
    const uint32_t lane = threadIdx.x & 63;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t r0 = (blockIdx.x * MM_WAVES + wave) * R;
    const uint32_t i0 = blockIdx.y * NBT;
    const uint32_t nb = min((uint32_t)NBT, p.n - i0);
    const uint32_t groups = p.cols / 32;
    float acc[NBT][R];
#pragma unroll
    for (int i = 0; i < NBT; i++)
#pragma unroll
        for (int r = 0; r < R; r++) acc[i][r] = 0.0f;
    // Rows past the matrix read its last row (their sums are never stored).
    const uint8_t* rowp[R];
#pragma unroll
    for (int r = 0; r < R; r++) rowp[r] = p.w + (size_t)min(r0 + r, p.rows - 1) * p.row_bytes;
    for (uint32_t t0 = 0; t0 < groups; t0 += TILE_GROUPS) {
        const uint32_t tg = min((uint32_t)TILE_GROUPS, groups - t0);
        // This lane's weights first, packed (lanes past the tile read its first group); then
        // the tile of every input row: float4 e of it is group e / 8, quarter e % 8.
        const uint32_t g = t0 + (lane < tg ? lane : 0u);
        uint32_t pk[R][PK<TY>];
#pragma unroll
        for (int r = 0; r < R; r++) group_load<TY>(rowp[r], g, pk[r]);
        __syncthreads();
        for (uint32_t e = threadIdx.x; e < nb * tg * 8; e += 64 * MM_WAVES) {
            const uint32_t i = e / (tg * 8), f = e % (tg * 8);
            const float4 v = *(const float4*)(p.x + (size_t)(i0 + i) * p.cols + 32 * t0 + 4 * f);
            *(float4*)&xs_dyn[i * TILE_GROUPS * XS + (f / 8) * XS + 4 * (f % 8)] = v;
        }
        __syncthreads();
        if (lane >= tg) continue;
        // One row's group against one input row's values (the same FMA order in both loop
        // nests below, so a row gets the same bits either way).
        auto dot = [&](const float (&q)[32], const float (&a)[2], const float (&b)[2], const float (&xv)[32],
                       float sx0, float sx1, float& acc_ir) {
            if constexpr (plain_type<TY>()) {
                float sum = acc_ir;
#pragma unroll
                for (int j = 0; j < 32; j++) sum = __builtin_fmaf(q[j], xv[j], sum);
                acc_ir = sum;
            } else {
                float s0 = 0.0f, s1 = 0.0f;
#pragma unroll
                for (int j = 0; j < 16; j++) {
                    s0 = __builtin_fmaf(q[j], xv[j], s0);
                    s1 = __builtin_fmaf(q[16 + j], xv[16 + j], s1);
                }
                float t = __builtin_fmaf(a[0], s0, acc_ir);
                t = __builtin_fmaf(a[1], s1, t);
                t = __builtin_fmaf(b[0], sx0, t);
                acc_ir = __builtin_fmaf(b[1], sx1, t);
            }
        };
        auto read_x = [&](int i, float (&xv)[32], float& sx0, float& sx1) {
#pragma unroll
            for (int k = 0; k < 8; k++) {
                const float4 v = *(const float4*)&xs_dyn[i * TILE_GROUPS * XS + lane * XS + 4 * k];
                xv[4 * k] = v.x; xv[4 * k + 1] = v.y; xv[4 * k + 2] = v.z; xv[4 * k + 3] = v.w;
            }
            sx0 = sx1 = 0.0f;
            if constexpr (!plain_type<TY>()) {
#pragma unroll
                for (int j = 0; j < 16; j++) {
                    sx0 += xv[j];
                    sx1 += xv[16 + j];
                }
            }
        };
        if constexpr (NBT == 1) {
            // One input row: its values once, each row unpacked in turn.
            float xv[32], sx0, sx1;
            read_x(0, xv, sx0, sx1);
#pragma unroll
            for (int r = 0; r < R; r++) {
                float q[32], a[2], b[2];
                group_unpack<TY>(pk[r], g, q, a, b);
                dot(q, a, b, xv, sx0, sx1, acc[0][r]);
            }
        } else {
            // A batch: each row unpacked once, the input rows' values read again from LDS.
            float sx[NBT][2];
#pragma unroll
            for (int i = 0; i < NBT; i++) {
                if (i < (int)nb) {
                    float xv[32];
                    read_x(i, xv, sx[i][0], sx[i][1]);
                }
            }
#pragma unroll
            for (int r = 0; r < R; r++) {
                float q[32], a[2], b[2];
                group_unpack<TY>(pk[r], g, q, a, b);
#pragma unroll
                for (int i = 0; i < NBT; i++) {
                    if (i < (int)nb) {
                        float xv[32], u0, u1;
                        read_x(i, xv, u0, u1);
                        dot(q, a, b, xv, sx[i][0], sx[i][1], acc[i][r]);
                    }
                }
            }
        }
    }
#pragma unroll
    for (int i = 0; i < NBT; i++) {
        if (i < (int)nb) {
#pragma unroll
            for (int r = 0; r < R; r++) {
                const float s = wave_sum(acc[i][r]);
                if (lane == 0 && r0 + r < p.rows) p.out[(size_t)(i0 + i) * p.rows + r0 + r] = s;
            }
        }
    }
}

template <uint32_t TY, int NBT, int R>
static void matmul_go(const MatmulParams& mp, hipStream_t s) {
    const uint32_t per_wg = MM_WAVES * R;
    const dim3 grid((mp.rows + per_wg - 1) / per_wg, (mp.n + NBT - 1) / NBT);
    const size_t lds = (size_t)min(mp.n, (uint32_t)NBT) * TILE_GROUPS * XS * sizeof(float);
    hipLaunchKernelGGL((k_matmul<TY, NBT, R>), grid, dim3(64 * MM_WAVES), lds, s, mp);
}

// One input row (decode): eight rows a wave when a group packs into at most 12 dwords and
// the matrix still gives 256+ workgroups (measured: the 14336 x 4096 Q4K product 21.3 ->
// 14.2 µs), else four. Batches: four rows a wave, eight input rows a pass.
template <uint32_t TY>
static hipError_t matmul_t(const MatmulParams& mp, hipStream_t s) {
    if (mp.n == 1) {
        if (PK<TY> <= 12 && mp.rows >= 256u * MM_WAVES * 8)
            matmul_go<TY, 1, (PK<TY> <= 12 ? 8 : 4)>(mp, s);
        else
            matmul_go<TY, 1, 4>(mp, s);
    } else {
        matmul_go<TY, NB, 4>(mp, s);
    }
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
