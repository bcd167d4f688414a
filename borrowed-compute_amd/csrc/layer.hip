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

// ---------------------------------------------------------------------------------------
// Batched product on the matrix cores (n >= MM_MIN input rows; the reference switches its
// batches to a matrix-unit product the same way, gpu/mod.rs:33-41, metal.rs:153-197).
// In the affine form, group g of weight row r is w = a q + b, q a small integer; so
// sum_k w x = a sum q x + b sum x. The MFMAs compute sum q x with x split into f16 parts,
// x = hi + lo 2^-12 (lo stored scaled by 2^12 so it keeps its 11 bits): about 22 bits,
// each product exact in f32, f32-level sums.
//
// k_matmul_mm: a workgroup is W waves of 16 weight rows, eight input rows and a K range of
// at most MM_K units of 256 columns. The range's x is staged once in LDS as 16 A rows: rows
// 0..7 the eight inputs' hi, rows 8..15 their lo, so one v_mfma_f32_16x16x32_f16 over group
// g gives D[i][l] = sum hi_i q (i < 8) and sum lo_{i-8} q (i >= 8) for the wave's 16 rows at
// once. Lane 16 c + l holds 8 weights of group g of row r0 + l (8c .. 8c + 7) as its B
// operand, unpacked from the ggml bytes in registers, in the order 0, 2, 1, 3, 4, 6, 5, 7
// (pairs of bytes 0, 2 and 1, 3 of a dword make the f16 pairs directly; staged x is
// permuted alike, and the MFMA's sum over k is the group's either way): each field is put
// under the f16 exponent of 1024 (one v_and_or_b32 for a pair of nibbles, v_perm_b32 for a
// pair of bytes) and one packed f16 subtraction takes 1024 and the format's fixed offset
// away (Q4_0 8, Q5_0 16, Q6K 32, Q8_0 -128 after a sign flip). D[4c + i][l] in lane
// 16 c + l: c < 2 the hi sums of input 4c + i, c >= 2 the lo sums of input 4(c - 2) + i;
// per group each lane adds a_eff D[i] (a_eff: a with the lo scale folded in) to four
// accumulators. The b sum x terms (Q4_1, Q5_1: m; Q4K, Q5K: -dmin m_j) are a product over
// groups of their own: a v_mfma_f32_16x16x4_f32 a half unit, A = the groups' sums of x
// (rows 8..15 zero), B = the groups' b, accumulated across the range. Q6K (a scale a 16 weights) takes two
// v_mfma_f32_16x16x16_f16 a group, one a half; F16 has no scale and chains its MFMAs
// through the accumulators. The units' bytes are loaded MM_PF units ahead. K splits: their
// number depends on rows and cols only; a split's partial is (hi + lo) + b terms of its
// units, and the row's result the splits' partials added in split order, whether one
// workgroup runs the splits one after another or ks workgroups run them at once and the
// last to finish (a device counter per tile) adds them: an input row's bits depend on that
// row alone, never on n or its place in the batch.
constexpr float MM_LO = 4096.0f;   // lo = (x - hi) * MM_LO
constexpr uint32_t MM_MIN = 2;     // batches of at least this many rows take the matrix cores (MM_FROM)
// Units (256 columns) a K split at most: the staged x takes 16 rows x (256 MM_K + 8) halves of
// LDS (the 8: 16-byte reads of 16 rows on distinct banks); the K-quants also pass each unit's
// bytes through LDS, so their splits are shorter.
template <uint32_t TY>
constexpr bool MM_LDSP = TY != G_F16;  // units pass through LDS (all block formats)
template <uint32_t TY>
constexpr uint32_t MM_K = MM_LDSP<TY> ? 4 : 8;
template <uint32_t TY>
constexpr uint32_t MM_XS = MM_K<TY> * 256 + 8;
constexpr uint32_t MM_PAR = MATMUL_COUNTERS;  // tiles (W x 16 rows x 8 inputs) up to which K splits run in parallel

template <uint32_t TY>
constexpr bool mm_type() {
    return TY == G_F16 || TY == G_Q8_0 || TY == G_Q4_0 || TY == G_Q4_1 || TY == G_Q5_0 || TY == G_Q5_1 ||
           TY == G_Q4K || TY == G_Q5K || TY == G_Q6K;
}
// Formats whose b sum x terms take the f32 MFMA.
template <uint32_t TY>
constexpr bool mm_sum() {
    return TY == G_Q4_1 || TY == G_Q5_1 || TY == G_Q4K || TY == G_Q5K;
}
// Dwords a lane loads of one unit (8 groups) of its row, and holds of it after mm_fix.
template <uint32_t TY>
constexpr int MW = TY == G_F16 ? 32 : TY == G_Q8_0 ? 20 : TY == G_Q6K ? 16 : 12;
template <uint32_t TY>
constexpr int MWD = TY == G_Q5K ? 14 : TY == G_Q6K ? 29 : MW<TY>;
// Units loaded ahead; waves a workgroup (eight where the registers allow four waves a SIMD).
template <uint32_t TY>
constexpr int MM_PF = 2;
template <uint32_t TY>
constexpr int MM_W = MM_LDSP<TY> ? 8 : 4;
// Bytes of a unit.
template <uint32_t TY>
constexpr uint32_t MM_UB = TY == G_F16 ? 512 : TY == G_Q8_0 ? 272 : TY == G_Q4_0 ? 144 : TY == G_Q4_1 ? 160
                         : TY == G_Q5_0 ? 176 : TY == G_Q5_1 ? 192 : TY == G_Q4K ? 144 : TY == G_Q5K ? 176 : 210;

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// The lane order of a dword's four bytes: 0, 2, 1, 3.
// Bytes of v as f16 values 1024 + b - off, in that order (two f16 pairs).
__device__ __forceinline__ u32x2 bytes_f16(uint32_t v, half2 off) {
    const uint32_t e0 = __builtin_amdgcn_perm(0x64646464u, v, 0x04020400u);  // (0x6400 | b0, 0x6400 | b2)
    const uint32_t e1 = __builtin_amdgcn_perm(0x64646464u, v, 0x04030401u);  // (0x6400 | b1, 0x6400 | b3)
    const half2 h0 = __builtin_bit_cast(half2, e0) - off, h1 = __builtin_bit_cast(half2, e1) - off;
    return u32x2{__builtin_bit_cast(uint32_t, h0), __builtin_bit_cast(uint32_t, h1)};
}
__device__ __forceinline__ half8 bytes8_f16(uint32_t v0, uint32_t v1, half2 off) {
    const u32x2 a = bytes_f16(v0, off), b = bytes_f16(v1, off);
    return __builtin_bit_cast(half8, u32x4{a[0], a[1], b[0], b[1]});
}
// The field under m (within each 16 bits: 0x000f000f, 0x00f000f0) of bytes 0, 2 of v as f16
// 1024 + f - off (exact): the field under the exponent of 1024 (one v_and_or_b32), then one
// packed subtraction. (Fields as f16 subnormals, f 2^-24, would need no subtraction, but the
// matrix cores multiply subnormals less exactly: about 1.7e-6 of a row's scale against 2e-7.)
// (v & m) | e in one v_and_or_b32 (m in a VGPR, e an SGPR: the instruction may read one
// SGPR and no literal, so the compiler otherwise splits it in two).
__device__ __forceinline__ uint32_t and_or(uint32_t v, uint32_t m, uint32_t e) {
    uint32_t r;
    asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(r) : "v"(v), "v"(m), "s"(e));
    return r;
}
__device__ __forceinline__ uint32_t field_pair(uint32_t v, uint32_t m, half2 off, uint32_t extra = 0u) {
    return __builtin_bit_cast(uint32_t, __builtin_bit_cast(half2, and_or(v, m, extra | 0x64006400u)) - off);
}
// As field_pair, times a scale in one packed FMA: (1024 + f) c1 + c2 with c2 = -1024 c1, exact
// while f c1 is an f16 integer (K-quant sub-block scale times field: at most 63 x 31).
__device__ __forceinline__ uint32_t field_pair_sc(uint32_t v, uint32_t m, half2 c1, half2 c2, uint32_t extra = 0u) {
    const half2 e = __builtin_bit_cast(half2, and_or(v, m, extra | 0x64006400u));
    return __builtin_bit_cast(uint32_t, __builtin_elementwise_fma(e, c1, c2));
}
// Bytes 0, 2, then 1, 3 of two dwords.
__device__ __forceinline__ half8 fields8(uint32_t v0, uint32_t v1, uint32_t m, half2 off) {
    return __builtin_bit_cast(half8, u32x4{field_pair(v0, m, off), field_pair(v0 >> 8, m, off),
                                           field_pair(v1, m, off), field_pair(v1 >> 8, m, off)});
}
// Four bits to bit 4 of bytes 0..3.
__device__ __forceinline__ uint32_t bit4_spread(uint32_t b4) { return ((b4 * 0x00204081u) & 0x01010101u) << 4; }
// Lane (c, row) loads of unit u (8 groups) of its row.
template <uint32_t TY>
__device__ __forceinline__ void mm_load(const uint8_t* __restrict__ row, uint32_t u, uint32_t c,
                                        uint32_t (&d)[MW<TY>]) {
    if constexpr (TY == G_F16) {
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const u32x4 v = *(const u32x4*)(row + (size_t)(8 * u + j) * 64 + 16 * c);
            d[4 * j] = v[0]; d[4 * j + 1] = v[1]; d[4 * j + 2] = v[2]; d[4 * j + 3] = v[3];
        }
    } else if constexpr (TY == G_Q8_0) {
        // Row-contiguous lane order as the K-quants' (below): 17 pieces a unit, lane quad q
        // takes pieces 4 l + (lane & 3), l < 5 (the repeats past the unit are its last piece).
        const uint8_t* bb = row + (size_t)u * 272;
        const uint32_t pq = threadIdx.x & 3u;
#pragma unroll
        for (int l = 0; l < 5; l++) {
            const u32x4 v = *(const u32x4*)(bb + 16 * min(4 * l + pq, 16u));
            d[4 * l] = v[0]; d[4 * l + 1] = v[1]; d[4 * l + 2] = v[2]; d[4 * l + 3] = v[3];
        }
    } else if constexpr (TY == G_Q4_0 || TY == G_Q4_1 || TY == G_Q5_0 || TY == G_Q5_1) {
        // row-contiguous lane order, as the K-quants' below (9 to 12 pieces a unit)
        constexpr uint32_t NP = MM_UB<TY> / 16;
        const uint8_t* bb = row + (size_t)u * MM_UB<TY>;
        const uint32_t pq = threadIdx.x & 3u;
#pragma unroll
        for (int l = 0; l < 3; l++) {
            const u32x4 v = *(const u32x4*)(bb + 16 * min(4 * l + pq, NP - 1));
            d[4 * l] = v[0]; d[4 * l + 1] = v[1]; d[4 * l + 2] = v[2]; d[4 * l + 3] = v[3];
        }
    } else if constexpr (TY == G_Q4K || TY == G_Q5K) {
        // Row-contiguous lane order (the memory path coalesces consecutive lanes: 64 bytes of
        // one row a lane quad), 16-byte pieces 4 l + (lane & 3) of the unit for l < 3 (the last
        // load's pieces past the unit repeat its last); `row` is the lane quad's row, and
        // mm_fix moves the pieces through LDS into the matrix-core layout.
        constexpr uint32_t NP = MM_UB<TY> / 16;  // pieces a unit: 9 (Q4K), 11 (Q5K)
        const uint8_t* bb = row + (size_t)u * MM_UB<TY>;
        const uint32_t pq = threadIdx.x & 3u;
#pragma unroll
        for (int l = 0; l < 3; l++) {
            const u32x4 v = *(const u32x4*)(bb + 16 * min(4 * l + pq, NP - 1));
            d[4 * l] = v[0]; d[4 * l + 1] = v[1]; d[4 * l + 2] = v[2]; d[4 * l + 3] = v[3];
        }
    } else {  // Q6K, row-contiguous lane order: the 16-byte pieces from the unit's start
        // rounded down to 16 (at most 14 pieces hold its 210 bytes; a lane quad takes pieces
        // 4 l + (lane & 3), l < 4, those past the last that holds unit bytes repeat it, so no
        // read leaves the 16-byte blocks the unit touches)
        const uint8_t* bb = row + (size_t)u * 210;
        const uintptr_t a0 = (uintptr_t)bb & ~(uintptr_t)15;
        const uint32_t km = (uint32_t)((uintptr_t)bb + 209 - a0) / 16, pq = threadIdx.x & 3u;
#pragma unroll
        for (int l = 0; l < 4; l++) {
            const u32x4 v = *(const u32x4*)(a0 + 16 * min(4 * l + pq, km));
            d[4 * l] = v[0]; d[4 * l + 1] = v[1]; d[4 * l + 2] = v[2]; d[4 * l + 3] = v[3];
        }
    }
}

// After a unit's loads land (K-quants): each lane quad's three pieces go to the wave's LDS
// rows (row q = lane / 4, the unit's 16-byte pieces, piece p at slot p ^ ((q >> 2) & 3) of a
// 192-byte row: the quads' 64-byte writes and the 16 rows' reads of one piece fall on
// distinct banks), and each lane reads back what the matrix-core layout gives it: the header
// (d, dmin, scales) and slice c of each 32-byte qs chunk (Q5K also qh bytes 8c .. 8c + 7),
// into d[0..3], d[4 + 2k..5 + 2k] (chunk k) and d[12..13].
// LDS bytes a row of a unit: K-quants 192 (swizzled pieces), Q8_0 272 (the unit as it is:
// a stride of 68 dwords puts the 16 rows' dword reads of one offset on distinct banks).
// The 32-weight formats' units keep their bytes as they are, in rows of an odd number of
// 16-byte pieces (Q4_1, Q5_1 padded by one) for the same bank spread.
template <uint32_t TY>
constexpr uint32_t MM_WT = TY == G_Q8_0 ? 272 : TY == G_Q6K ? 240 : TY == G_Q4_0 ? 144 : TY == G_Q4_1 ? 176
                         : TY == G_Q5_0 ? 176 : TY == G_Q5_1 ? 208 : 192;
// s: the lane's loads; d: what mm_unit and mm_group read; sq, sm: the lane quad's and the
// lane's own row's unit start modulo 16 (Q6K).
template <uint32_t TY>
__device__ __forceinline__ void mm_fix(const uint32_t (&s)[MW<TY>], uint32_t (&d)[MWD<TY>], uint8_t* wt, uint32_t c,
                                       uint32_t rl, uint32_t sq, uint32_t sm) {
    if constexpr (!MM_LDSP<TY>) {
#pragma unroll
        for (int k = 0; k < MW<TY>; k++) d[k] = s[k];
    }
    if constexpr (TY == G_Q8_0 || TY == G_Q4_0 || TY == G_Q4_1 || TY == G_Q5_0 || TY == G_Q5_1) {
        // the unit to the LDS rows as it is; mm_group reads each group from there
        constexpr uint32_t NP = MM_UB<TY> / 16;
        const uint32_t q = (threadIdx.x & 63u) >> 2, pq = threadIdx.x & 3u;
#pragma unroll
        for (int l = 0; l < MW<TY> / 4; l++)
            if (4 * l + pq < NP)
                *(u32x4*)(wt + q * MM_WT<TY> + 16 * (4 * l + pq)) = u32x4{s[4 * l], s[4 * l + 1], s[4 * l + 2], s[4 * l + 3]};
        if constexpr (TY == G_Q4_1 || TY == G_Q5_1) {  // m of groups c and 4 + c (the b terms)
            constexpr uint32_t BS = TY == G_Q4_1 ? 20 : 24;
            const uint8_t* rw = wt + rl * MM_WT<TY>;
            d[0] = *(const uint16_t*)(rw + BS * c + 2);
            d[1] = *(const uint16_t*)(rw + BS * (4 + c) + 2);
        }
    }
    if constexpr (TY == G_Q6K) {
        // pieces to the LDS rows as loaded (unit byte b at sq + b of the quad's row); then the
        // lane reads, from its own row (byte b at sm + b), the dwords the unpacking takes: at 4c
        // and 16 + 4c (two each) of the six 32-byte ql / qh runs, and bytes 192..209 (scales, d),
        // all from the dword-aligned base of the unit's start
        const uint32_t q = (threadIdx.x & 63u) >> 2, pq = threadIdx.x & 3u, kq = (sq + 209) / 16;
#pragma unroll
        for (int l = 0; l < 4; l++)
            if (4 * l + pq <= kq)
                *(u32x4*)(wt + q * 240 + 16 * (4 * l + pq)) = u32x4{s[4 * l], s[4 * l + 1], s[4 * l + 2], s[4 * l + 3]};
        const uint8_t* a = wt + rl * 240 + (sm & ~3u);
#pragma unroll
        for (int k = 0; k < 6; k++) {
            const uint32_t o = k < 4 ? 32 * k : 128 + 32 * (k - 4);
            d[4 * k] = *(const uint32_t*)(a + o + 4 * c);
            d[4 * k + 1] = *(const uint32_t*)(a + o + 4 * c + 4);
            d[4 * k + 2] = *(const uint32_t*)(a + o + 16 + 4 * c);
            d[4 * k + 3] = *(const uint32_t*)(a + o + 20 + 4 * c);
        }
#pragma unroll
        for (int k = 0; k < 5; k++) d[24 + k] = *(const uint32_t*)(a + 192 + 4 * k);
    }
    if constexpr (TY == G_Q4K || TY == G_Q5K) {
        constexpr uint32_t NP = MM_UB<TY> / 16, QP = TY == G_Q4K ? 1 : 3;  // pieces; first qs piece
        const uint32_t q = (threadIdx.x & 63u) >> 2, pq = threadIdx.x & 3u, fq = (q >> 2) & 3u;
#pragma unroll
        for (int l = 0; l < 3; l++)
            if (4 * l + pq < NP)  // (the last load's repeats of the unit's last piece stay out)
                *(u32x4*)(wt + q * MM_WT<TY> + 16 * ((4 * l + pq) ^ fq)) = u32x4{s[4 * l], s[4 * l + 1], s[4 * l + 2], s[4 * l + 3]};
        const uint8_t* rw = wt + rl * MM_WT<TY>;
        const uint32_t fr = (rl >> 2) & 3u;
        const u32x4 h = *(const u32x4*)(rw + 16 * fr);
        d[0] = h[0]; d[1] = h[1]; d[2] = h[2]; d[3] = h[3];
#pragma unroll
        for (int k = 0; k < 4; k++) {
            const u32x2 v = *(const u32x2*)(rw + 16 * ((QP + 2 * k + (c >> 1)) ^ fr) + 8 * (c & 1));
            d[4 + 2 * k] = v[0];
            d[5 + 2 * k] = v[1];
        }
        if constexpr (TY == G_Q5K) {
            const u32x2 v = *(const u32x2*)(rw + 16 * ((1 + (c >> 1)) ^ fr) + 8 * (c & 1));
            d[12] = v[0];
            d[13] = v[1];
        }
    }
}

// What a unit's groups share: the scale factors and packed scale bytes (K-quants), and the
// lane's two b values (groups c and 4 + c: B of the f32 MFMAs).
struct MMUnit {
    float dl = 0.0f, b0 = 0.0f, b1 = 0.0f;
    uint32_t scA = 0, scB = 0;
};

template <uint32_t TY>
__device__ __forceinline__ MMUnit mm_unit(const uint32_t (&d)[MWD<TY>], uint32_t c, float fl) {
    MMUnit m;
    if constexpr (TY == G_Q4K || TY == G_Q5K) {
        // scale and min bytes of sub-blocks 0..3 and 4..7 (6 bits each, quant.rs:136-146)
        const uint32_t s0 = d[1], s1 = d[2], s2 = d[3];
        m.scA = s0 & 0x3f3f3f3fu;
        m.scB = (s2 & 0x0f0f0f0fu) | ((s0 >> 2) & 0x30303030u);
        const uint32_t mnA = s1 & 0x3f3f3f3fu, mnB = ((s2 >> 4) & 0x0f0f0f0fu) | ((s1 >> 2) & 0x30303030u);
        const float dd = h2f(d[0] & 0xffffu) * fl, ndm = -h2f(d[0] >> 16);
        m.dl = dd;
        m.b0 = ndm * (float)((mnA >> (8 * c)) & 255u);
        m.b1 = ndm * (float)((mnB >> (8 * c)) & 255u);
    } else if constexpr (TY == G_Q4_1 || TY == G_Q5_1) {
        m.b0 = h2f(d[0]);
        m.b1 = h2f(d[1]);
    }
    return m;
}

// Group j of a loaded unit for lane c: B operand(s) and a (fl and the field scale folded in).
// Q6K gives two half operands q4[0], q4[1] (16x16x16 MFMAs) and a0, a1.
template <uint32_t TY>
__device__ __forceinline__ void mm_group(const uint32_t (&d)[MWD<TY>], const MMUnit& m, const uint8_t* unit_base,
                                         const uint8_t* rw, int j, uint32_t c, float fl, half8& q, half4 (&q4)[2],
                                         float& a0, float& a1) {
    if constexpr (TY == G_F16) {  // weights 8c .. 8c + 7 in order (x staged unpermuted)
        q = __builtin_bit_cast(half8, u32x4{d[4 * j], d[4 * j + 1], d[4 * j + 2], d[4 * j + 3]});
    } else if constexpr (TY == G_Q8_0) {  // from the lane's LDS row rw (the unit, 16-aligned)
        const uint32_t b = 34 * j + 2 + 8 * c, a = b & ~3u, sh = b & 3u;  // qs bytes 8c .. of block j
        const uint32_t w[3] = {*(const uint32_t*)(rw + a), *(const uint32_t*)(rw + a + 4),
                               *(const uint32_t*)(rw + a + 4 + 2 * sh)};
        const uint32_t w0 = __builtin_amdgcn_alignbyte(w[1], w[0], sh), w1 = __builtin_amdgcn_alignbyte(w[2], w[1], sh);
        q = bytes8_f16(w0 ^ 0x80808080u, w1 ^ 0x80808080u, half2{(f16)1152.0f, (f16)1152.0f});
        a0 = h2f(*(const uint16_t*)(rw + 34 * j)) * fl;
    } else if constexpr (TY == G_Q4_0 || TY == G_Q5_0) {
        // from the lane's LDS row rw; lanes 0, 1: low nibbles, lanes 2, 3: high nibbles
        // (weights 16 ..), as q - 8 (Q4_0) or, with qh byte c as bit 4, q - 16 (Q5_0)
        constexpr uint32_t BS = TY == G_Q4_0 ? 18 : 22, QS = TY == G_Q4_0 ? 2 : 6;
        const uint32_t b = BS * j + QS + 8 * (c & 1), a = b & ~3u, sh = b & 3u;
        const uint32_t w[3] = {*(const uint32_t*)(rw + a), *(const uint32_t*)(rw + a + 4),
                               *(const uint32_t*)(rw + a + 4 + 2 * sh)};
        uint32_t w0 = __builtin_amdgcn_alignbyte(w[1], w[0], sh), w1 = __builtin_amdgcn_alignbyte(w[2], w[1], sh);
        const uint32_t ns = c < 2 ? 0u : 4u;
        if constexpr (TY == G_Q4_0) {
            q = fields8(w0 >> ns, w1 >> ns, 0x000f000fu, half2{(f16)1032.0f, (f16)1032.0f});
        } else {
            const uint32_t qh = *(const uint8_t*)(rw + BS * j + 2 + c);  // bit 4 of weights 8c ..
            w0 = ((w0 >> ns) & 0x0f0f0f0fu) | bit4_spread(qh & 15u);
            w1 = ((w1 >> ns) & 0x0f0f0f0fu) | bit4_spread(qh >> 4);
            q = bytes8_f16(w0, w1, half2{(f16)1040.0f, (f16)1040.0f});
        }
        a0 = h2f(*(const uint16_t*)(rw + BS * j)) * fl;
    } else if constexpr (TY == G_Q4_1 || TY == G_Q5_1) {  // from the lane's LDS row rw
        constexpr uint32_t BS = TY == G_Q4_1 ? 20 : 24, QS = TY == G_Q4_1 ? 4 : 8;
        const uint8_t* g = rw + BS * j;
        const uint32_t x0 = *(const uint32_t*)(g + QS + 8 * (c & 1)), x1 = *(const uint32_t*)(g + QS + 8 * (c & 1) + 4);
        const uint32_t ns = c < 2 ? 0u : 4u;
        if constexpr (TY == G_Q4_1) {
            q = fields8(x0 >> ns, x1 >> ns, 0x000f000fu, half2{(f16)1024.0f, (f16)1024.0f});
        } else {
            const uint32_t qh = g[4 + c];  // qh byte c
            const uint32_t w0 = ((x0 >> ns) & 0x0f0f0f0fu) | bit4_spread(qh & 15u);
            const uint32_t w1 = ((x1 >> ns) & 0x0f0f0f0fu) | bit4_spread(qh >> 4);
            q = bytes8_f16(w0, w1, half2{(f16)1024.0f, (f16)1024.0f});
        }
        a0 = h2f(*(const uint16_t*)g) * fl;
    } else if constexpr (TY == G_Q4K || TY == G_Q5K) {
        const int k = j / 2, hi = j % 2;
        const uint32_t v0 = d[4 + 2 * k], v1 = d[5 + 2 * k];
        // B = q sc_j (an f16 integer): the sub-block scale rides in the unpacking FMA, so the
        // unit's eight MFMAs chain through one accumulator and d scales the unit once.
        // (sc_j, sc_j) from its byte under the exponent of 1024: (1024 + sc) s - 1024 s, with
        // s = 1/16 for Q4K's high nibbles, which stay in place (16 q).
        const uint32_t b = (uint32_t)(j % 4);
        const half2 e = __builtin_bit_cast(half2, __builtin_amdgcn_perm(0x64646464u, j < 4 ? m.scA : m.scB,
                                                                        0x04000400u | b | (b << 16)));
        const f16 s16 = (TY == G_Q4K && hi) ? (f16)0.0625f : (f16)1.0f;
        const half2 c1 = __builtin_elementwise_fma(e, half2{s16, s16}, half2{(f16)-1024.0f * s16, (f16)-1024.0f * s16});
        const half2 c2 = c1 * half2{(f16)-1024.0f, (f16)-1024.0f};
        if constexpr (TY == G_Q4K) {
            const uint32_t mk = hi ? 0x00f000f0u : 0x000f000fu;
            q = __builtin_bit_cast(half8, u32x4{field_pair_sc(v0, mk, c1, c2), field_pair_sc(v0 >> 8, mk, c1, c2),
                                                field_pair_sc(v1, mk, c1, c2), field_pair_sc(v1 >> 8, mk, c1, c2)});
        } else {  // bit j of qh byte t is bit 4 of weight t
            const uint32_t h0 = d[12] >> j, h1 = d[13] >> j;
            const uint32_t n0 = hi ? v0 >> 4 : v0, n1 = hi ? v1 >> 4 : v1;
            const uint32_t m4 = 0x000f000fu, b4 = 0x00010001u;
            q = __builtin_bit_cast(half8, u32x4{field_pair_sc(n0, m4, c1, c2, (h0 & b4) << 4),
                                                field_pair_sc(n0 >> 8, m4, c1, c2, ((h0 >> 8) & b4) << 4),
                                                field_pair_sc(n1, m4, c1, c2, (h1 & b4) << 4),
                                                field_pair_sc(n1 >> 8, m4, c1, c2, ((h1 >> 8) & b4) << 4)});
        }
    } else {  // Q6K
        const int hh = j / 4, qr = j % 4, s = qr & 1;
        const uint32_t sh = (uint32_t)((uintptr_t)unit_base & 3u);
        // lane c: weights 4c .. 4c + 3 (half 0) and 16 + 4c .. (half 1) of the group
        const uint32_t* L = &d[4 * (2 * hh + s)];
        const uint32_t* H = &d[4 * (4 + hh)];
        const uint32_t l0 = __builtin_amdgcn_alignbyte(L[1], L[0], sh), l1 = __builtin_amdgcn_alignbyte(L[3], L[2], sh);
        const uint32_t h0 = __builtin_amdgcn_alignbyte(H[1], H[0], sh), h1 = __builtin_amdgcn_alignbyte(H[3], H[2], sh);
        const uint32_t ns = qr < 2 ? 0u : 4u;
        const uint32_t v0 = ((l0 >> ns) & 0x0f0f0f0fu) | (((h0 >> (2 * qr)) & 0x03030303u) << 4);
        const uint32_t v1 = ((l1 >> ns) & 0x0f0f0f0fu) | (((h1 >> (2 * qr)) & 0x03030303u) << 4);
        const half2 o = half2{(f16)1056.0f, (f16)1056.0f};
        q4[0] = __builtin_bit_cast(half4, bytes_f16(v0, o));
        q4[1] = __builtin_bit_cast(half4, bytes_f16(v1, o));
        // scales (int8) 8 hh + 2 qr and + 1, d: bytes 192 .. 209 of the block
        const uint32_t sw = __builtin_amdgcn_alignbyte(d[25 + hh * 2 + (qr >> 1)], d[24 + hh * 2 + (qr >> 1)], sh);
        const uint32_t sp = sw >> (16 * (qr & 1));  // bytes 2 qr, 2 qr + 1 of the 4-byte window
        const uint32_t dw = __builtin_amdgcn_alignbyte(d[28], d[28], sh) & 0xffffu;  // d: bytes 208, 209
        const float dd = h2f(dw) * fl;
        a0 = dd * (float)(int8_t)(uint8_t)(sp & 255u);
        a1 = dd * (float)(int8_t)(uint8_t)((sp >> 8) & 255u);
    }
}

struct MMParams {
    const uint8_t* w;
    const float* x;
    float* out;
    float* part;    // [ks][npad][rows]: parallel splits' partials
    uint32_t* cnt;  // [tiles]: arrivals of a tile's parallel splits (zero between calls)
    uint32_t rows, cols, n, npad, row_bytes, units, ks, par;
};

template <uint32_t TY>
__global__ __launch_bounds__(64 * MM_W<TY>, MM_W<TY> / 2) void k_matmul_mm(const MMParams p) {  // two workgroups a CU
    constexpr bool SUM = mm_sum<TY>(), KP = TY != G_F16;
    constexpr int PF = MM_PF<TY>, W = MM_W<TY>, NT = 64 * W;
    constexpr uint32_t XS = MM_XS<TY>;
    __shared__ __attribute__((aligned(16))) f16 xs[16 * XS];
    __shared__ __attribute__((aligned(16))) float ss[SUM ? MM_K<TY> * 8 * 16 : 4];
    constexpr bool KQ = MM_LDSP<TY>;  // units pass through LDS (mm_fix)
    __shared__ __attribute__((aligned(16))) uint8_t wtb[KQ ? W * 16 * MM_WT<TY> : 16];
    __shared__ uint32_t last;
    const uint32_t tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const uint32_t c = lane >> 4, rl = lane & 15;
    const uint32_t r0 = blockIdx.x * (16 * W) + 16 * w, r = r0 + rl, i0 = blockIdx.y * 8;
    const bool live = r0 < p.rows;  // the wave has rows
    // the rows a lane loads: its matrix-core row (mrowp), or (KQ) its lane quad's
    const uint8_t* mrowp = p.w + (size_t)min(r, p.rows - 1) * p.row_bytes;
    const uint8_t* rowp = KQ ? p.w + (size_t)min(r0 + (lane >> 2), p.rows - 1) * p.row_bytes : mrowp;
    uint8_t* wt = wtb + (KQ ? w * 16 * MM_WT<TY> : 0);
    const float fl = c >= 2 ? 1.0f / MM_LO : 1.0f;
    const uint32_t kz0 = p.par ? blockIdx.z : 0, kz1 = p.par ? blockIdx.z + 1 : p.ks;
    float tot[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    for (uint32_t kz = kz0; kz < kz1; kz++) {
        const uint32_t ua = kz * p.units / p.ks, nu = (kz + 1) * p.units / p.ks - ua;
        // Every step loads one unit (past the range's end its last unit again), so the loads
        // outstanding at each use are the same and the compiler's waits stay partial.
        uint32_t pk[PF][MW<TY>];
        if (live) {
#pragma unroll
            for (int f = 0; f < PF; f++) mm_load<TY>(rowp, ua + min((uint32_t)f, nu - 1), c, pk[f]);
        }
        if (kz != kz0) __syncthreads();  // every wave is done with the previous split's x
        // Stage x: float4 q of the range (input q / (64 nu), columns 4 (q % (64 nu)) ..), read
        // coalesced (consecutive lanes, consecutive 16 bytes), as hi and lo in the lanes' k order
        // (within each 8 columns: 0, 2, 1, 3, 4, 6, 5, 7, so a float4's four values stay
        // together); (SUM) a group's sum over the 8 lanes that hold it, in a fixed tree.
        const uint32_t q4 = 64 * nu;  // float4s an input row of the range
        constexpr int XB = W == 8 ? 4 : 8;  // loads in flight a thread (eight waves: a split's all)
        for (uint32_t q0 = tid; q0 < 8 * q4; q0 += XB * NT) {
            float4 v[XB];
#pragma unroll
            for (int t = 0; t < XB; t++) {
                const uint32_t q = q0 + t * NT, in = i0 + q / q4;
                v[t] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
                if (q < 8 * q4 && in < p.n)
                    v[t] = *(const float4*)(p.x + (size_t)in * p.cols + (size_t)ua * 256 + 4 * (q % q4));
            }
#pragma unroll
            for (int t = 0; t < XB; t++) {
                const uint32_t q = q0 + t * NT, i = q / q4, cq = q % q4;
                if (q >= 8 * q4) break;  // uniform: 8 q4 is a multiple of NT
                if constexpr (SUM) {
                    float sg = ((v[t].x + v[t].y) + v[t].z) + v[t].w;
                    sg += __shfl_xor(sg, 1, 64);
                    sg += __shfl_xor(sg, 2, 64);
                    sg += __shfl_xor(sg, 4, 64);
                    if ((cq & 7) == 0) {
                        ss[(cq / 8) * 16 + i] = sg;
                        ss[(cq / 8) * 16 + 8 + i] = 0.0f;
                    }
                }
                const float xs4[4] = {v[t].x, KP ? v[t].z : v[t].y, KP ? v[t].y : v[t].z, v[t].w};
                half4 h, l;
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    const f16 hv = (f16)xs4[e];
                    h[e] = hv;
                    l[e] = (f16)((xs4[e] - (float)hv) * MM_LO);
                }
                *(half4*)&xs[i * XS + 4 * cq] = h;
                *(half4*)&xs[(8 + i) * XS + 4 * cq] = l;
            }
        }
        __syncthreads();
        f32x4 acc = f32x4{0.0f, 0.0f, 0.0f, 0.0f}, accb = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
        if (live) {
            for (uint32_t u0 = 0; u0 < nu; u0 += PF) {
#pragma unroll
                for (int f = 0; f < PF; f++) {
                    const uint32_t lu = u0 + f;
                    if (lu < nu) {
                        const uint8_t* ub = mrowp + (size_t)(ua + lu) * MM_UB<TY>;  // the lane's row's unit
                        const uint8_t* qb = rowp + (size_t)(ua + lu) * MM_UB<TY>;   // its lane quad's
                        uint32_t dd[MWD<TY>];
                        mm_fix<TY>(pk[f], dd, wt, c, rl, (uint32_t)((uintptr_t)qb & 15u), (uint32_t)((uintptr_t)ub & 15u));
                        const MMUnit m = mm_unit<TY>(dd, c, fl);
                        if constexpr (SUM) {  // sum_g b_g s_g over the unit's groups, 4 at a time
                            const float s0 = ss[(lu * 8 + c) * 16 + rl], s1 = ss[(lu * 8 + 4 + c) * 16 + rl];
                            accb = __builtin_amdgcn_mfma_f32_16x16x4f32(s0, m.b0, accb, 0, 0, 0);
                            accb = __builtin_amdgcn_mfma_f32_16x16x4f32(s1, m.b1, accb, 0, 0, 0);
                        }
                        f32x4 accu = f32x4{0.0f, 0.0f, 0.0f, 0.0f}, accu2 = accu;  // even, odd groups
#pragma unroll
                        for (int j = 0; j < 8; j++) {
                            const uint32_t col = lu * 256 + 32 * j;
                            half8 q;
                            half4 q4[2];
                            float a0 = 0.0f, a1 = 0.0f;
                            mm_group<TY>(dd, m, ub, wt + rl * MM_WT<TY>, j, c, fl, q, q4, a0, a1);
                            if constexpr (TY == G_Q4K || TY == G_Q5K) {
                                const half8 xa = *(const half8*)&xs[rl * XS + col + 8 * c];
                                if (j % 2 == 0) accu = mfma16(xa, q, accu);
                                else accu2 = mfma16(xa, q, accu2);
                            } else if constexpr (TY == G_F16) {
                                const half8 xa = *(const half8*)&xs[rl * XS + col + 8 * c];
                                acc = mfma16(xa, q, acc);
                            } else if constexpr (TY == G_Q6K) {
                                const half4 x0 = *(const half4*)&xs[rl * XS + col + 4 * c];
                                const half4 x1 = *(const half4*)&xs[rl * XS + col + 16 + 4 * c];
                                const f32x4 z = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
                                const f32x4 d0 = __builtin_amdgcn_mfma_f32_16x16x16f16(x0, q4[0], z, 0, 0, 0);
                                const f32x4 d1 = __builtin_amdgcn_mfma_f32_16x16x16f16(x1, q4[1], z, 0, 0, 0);
#pragma unroll
                                for (int i = 0; i < 4; i++) acc[i] = __builtin_fmaf(a1, d1[i], __builtin_fmaf(a0, d0[i], acc[i]));
                            } else {
                                const half8 xa = *(const half8*)&xs[rl * XS + col + 8 * c];
                                const f32x4 dv = mfma16(xa, q, f32x4{0.0f, 0.0f, 0.0f, 0.0f});
#pragma unroll
                                for (int i = 0; i < 4; i++) acc[i] = __builtin_fmaf(a0, dv[i], acc[i]);
                            }
                        }
                        if constexpr (TY == G_Q4K || TY == G_Q5K) {
#pragma unroll
                            for (int i = 0; i < 4; i++) acc[i] = __builtin_fmaf(m.dl, accu[i] + accu2[i], acc[i]);
                        }
                    }
                    // the unit's registers are free: load into them directly (a load hoisted
                    // above their last use would land in other registers and wait to be copied)
                    __builtin_amdgcn_sched_barrier(0);
                    mm_load<TY>(rowp, ua + min(lu + PF, nu - 1), c, pk[f]);
                }
            }
        }
        if constexpr (TY == G_F16) {
#pragma unroll
            for (int i = 0; i < 4; i++) acc[i] *= fl;
        }
        // the split's partial in lanes c < 2 (input 4c + i): hi + lo, then the b terms; then
        // the splits in order
#pragma unroll
        for (int i = 0; i < 4; i++) {
            float pt = acc[i] + __shfl_xor(acc[i], 32, 64);
            if constexpr (SUM) pt += accb[i];
            tot[i] = kz == kz0 ? pt : tot[i] + pt;
        }
    }
    if (!p.par) {
        if (c < 2 && r < p.rows) {
#pragma unroll
            for (int i = 0; i < 4; i++)
                if (i0 + 4 * c + i < p.n) p.out[(size_t)(i0 + 4 * c + i) * p.rows + r] = tot[i];
        }
        return;
    }
    // Parallel splits: the partial to device memory (write-through stores), then the tile's
    // arrival count; the last workgroup of the tile adds the partials in split order.
    if (c < 2 && r < p.rows) {
#pragma unroll
        for (int i = 0; i < 4; i++)
            __hip_atomic_store(&p.part[((size_t)blockIdx.z * p.npad + i0 + 4 * c + i) * p.rows + r], tot[i],
                               __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __builtin_amdgcn_s_waitcnt(0);  // this thread's stores are done
    __syncthreads();
    const uint32_t tile = blockIdx.y * gridDim.x + blockIdx.x;
    if (tid == 0) {
        const uint32_t old = __hip_atomic_fetch_add(&p.cnt[tile], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        last = old == p.ks - 1;
    }
    __syncthreads();
    if (!last) return;
    // The tile's 8 x 16 W outputs, two a thread; eight splits' loads in flight at a time.
    const size_t stride = (size_t)p.npad * p.rows;
    float sum[2] = {0.0f, 0.0f};
    bool ok[2];
    const float* src[2];
#pragma unroll
    for (int h = 0; h < 2; h++) {
        const uint32_t e = tid + h * NT, rr = blockIdx.x * (16 * W) + e % (16 * W), in = i0 + e / (16 * W);
        ok[h] = rr < p.rows && in < p.n;
        src[h] = p.part + (size_t)min(in, p.npad - 1) * p.rows + min(rr, p.rows - 1);
    }
    for (uint32_t k0 = 0; k0 < p.ks; k0 += 8) {
        float v[2][8];
#pragma unroll
        for (int h = 0; h < 2; h++)
#pragma unroll
            for (int t = 0; t < 8; t++)
                v[h][t] = k0 + t < p.ks ? __hip_atomic_load(src[h] + (k0 + t) * stride, __ATOMIC_RELAXED,
                                                             __HIP_MEMORY_SCOPE_AGENT)
                                        : 0.0f;
#pragma unroll
        for (int h = 0; h < 2; h++)
#pragma unroll
            for (int t = 0; t < 8; t++)
                if (k0 + t < p.ks) sum[h] = k0 + t == 0 ? v[h][t] : sum[h] + v[h][t];
    }
#pragma unroll
    for (int h = 0; h < 2; h++) {
        const uint32_t e = tid + h * NT, rr = blockIdx.x * (16 * W) + e % (16 * W), in = i0 + e / (16 * W);
        if (ok[h]) p.out[(size_t)in * p.rows + rr] = sum[h];
    }
    if (tid == 0) __hip_atomic_store(&p.cnt[tile], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Rows a workgroup of the format takes.
static uint32_t mm_rows(uint32_t type) {
    return type == G_F16 ? 16 * MM_W<G_F16> : 16 * MM_W<G_Q4K>;
}
// K splits of a product: about two workgroups a CU from the rows alone (never from n), each
// split at most MM_K units.
static uint32_t mm_ks(uint32_t type, uint32_t rows, uint32_t cols) {
    const uint32_t rt = (rows + mm_rows(type) - 1) / mm_rows(type), units = cols / 256;
    const uint32_t kmax = type == G_F16 ? MM_K<G_F16> : MM_K<G_Q4K>;
    uint32_t ks = max(512u / rt, 1u);
    ks = max(ks, (units + kmax - 1) / kmax);
    ks = min(ks, units);
    return max(ks, 1u);
}
static bool mm_par(uint32_t type, uint32_t rows, uint32_t cols, uint32_t n) {
    const uint32_t rt = (rows + mm_rows(type) - 1) / mm_rows(type), nt = (n + 7) / 8;
    return mm_ks(type, rows, cols) > 1 && (uint64_t)rt * nt <= MM_PAR;
}

bool matmul_uses_mm(uint32_t type, uint32_t cols, uint32_t n) {
    switch (type) {
        case G_F16: case G_Q8_0: case G_Q4_0: case G_Q4_1: case G_Q5_0: case G_Q5_1: case G_Q4K: case G_Q5K:
        case G_Q6K: return n >= MM_MIN && cols % 256 == 0;
        default: return false;
    }
}

size_t matmul_scratch_bytes(uint32_t type, uint32_t rows, uint32_t cols, uint32_t n) {
    if (!matmul_uses_mm(type, cols, n) || !mm_par(type, rows, cols, n)) return 0;
    return (size_t)mm_ks(type, rows, cols) * ((n + 7) / 8 * 8) * rows * sizeof(float);
}

template <uint32_t TY>
static hipError_t matmul_mm_go(const MatmulParams& mp, void* scratch, uint32_t* counters, hipStream_t s) {
    const uint32_t ks = mm_ks(TY, mp.rows, mp.cols), rt = (mp.rows + 16 * MM_W<TY> - 1) / (16 * MM_W<TY>);
    const uint32_t nt = (mp.n + 7) / 8;
    const bool par = mm_par(TY, mp.rows, mp.cols, mp.n);
    if (par && (!scratch || !counters)) return hipErrorInvalidValue;
    const MMParams q{mp.w, mp.x, mp.out, (float*)scratch, counters, mp.rows, mp.cols, mp.n, nt * 8, mp.row_bytes,
                     mp.cols / 256, ks, par ? 1u : 0u};
    hipLaunchKernelGGL((k_matmul_mm<TY>), dim3(rt, nt, par ? ks : 1), dim3(64 * MM_W<TY>), 0, s, q);
    return hipGetLastError();
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
static hipError_t matmul_t(const MatmulParams& mp, void* scratch, uint32_t* counters, hipStream_t s) {
    if constexpr (mm_type<TY>()) {
        if (matmul_uses_mm(TY, mp.cols, mp.n)) return matmul_mm_go<TY>(mp, scratch, counters, s);
    }
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
                         uint32_t n, uint32_t row_bytes, void* scratch, uint32_t* counters, hipStream_t s) {
    const MatmulParams mp{(const uint8_t*)w, x, out, rows, cols, n, row_bytes};
    switch (type) {
        case G_F32: return matmul_t<G_F32>(mp, scratch, counters, s);
        case G_F16: return matmul_t<G_F16>(mp, scratch, counters, s);
        case G_BF16: return matmul_t<G_BF16>(mp, scratch, counters, s);
        case G_Q4_0: return matmul_t<G_Q4_0>(mp, scratch, counters, s);
        case G_Q4_1: return matmul_t<G_Q4_1>(mp, scratch, counters, s);
        case G_Q5_0: return matmul_t<G_Q5_0>(mp, scratch, counters, s);
        case G_Q5_1: return matmul_t<G_Q5_1>(mp, scratch, counters, s);
        case G_Q8_0: return matmul_t<G_Q8_0>(mp, scratch, counters, s);
        case G_Q4K: return matmul_t<G_Q4K>(mp, scratch, counters, s);
        case G_Q5K: return matmul_t<G_Q5K>(mp, scratch, counters, s);
        case G_Q6K: return matmul_t<G_Q6K>(mp, scratch, counters, s);
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
