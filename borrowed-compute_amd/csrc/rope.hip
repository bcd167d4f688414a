// RoPE, and RoPE fused with the KV-cache append.
//
// bc_rope: bc-infer's k_rope (crates/bc-infer/src/gpu/kernels.h:235-248, entry
// cuda.cu:81): pair i of every head of row r turns by theta = (f32)positions[r] *
// inv_freq[i], neox pairs (i, i + rope_dim/2), else (2i, 2i+1); x0' = x0 cos - x1 sin,
// x1' = x0 sin + x1 cos, each product rounded on its own as model.rs:395-400 does. The
// reference's CUDA path reduces theta by hand before a fast sine (cuda.cu:61-72) since
// angles reach tens of thousands of radians; here sincosf is the device library's
// full-range one.
//
// bc_rope_append: the four launches k_rope(q), k_rope(k), k_copy(k -> kc @ slot0*kvd),
// k_copy(v -> vc) of gpu/mod.rs:464-475 as one: each thread takes one pair of one head of
// one row, over the q heads (rotated in place), the k heads (rotated and stored into the
// cache, converted to its type) and the v heads (stored). The ragged form puts each row at a
// slot of its own: one new token of each of several conversations in one cache pool (the
// streams of crates/bc-mesh/src/engine.rs:25, 305-314, each appended by its own k_copy today).
#include "common.hpp"
#include "internal.hpp"

#include <math.h>

namespace bchip {

__global__ __launch_bounds__(256) void k_rope(float* __restrict__ x, const float* __restrict__ inv_freq,
                                              const uint32_t* __restrict__ positions, uint32_t rows,
                                              uint32_t heads, uint32_t hd, uint32_t rope_dim, uint32_t neox) {
    const uint32_t hh = rope_dim / 2;
    const uint64_t idx = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= (uint64_t)rows * heads * hh) return;
    const uint32_t i = idx % hh, h = (idx / hh) % heads;
    const uint64_t r = idx / ((uint64_t)hh * heads);
    float* hp = x + (r * heads + h) * hd;
    const float theta = (float)positions[r] * inv_freq[i];
    const uint32_t a = neox ? i : 2 * i, b = neox ? i + hh : 2 * i + 1;
    float y0, y1;
    rotate(hp[a], hp[b], theta, y0, y1);
    hp[a] = y0;
    hp[b] = y1;
}

// Cache slots of the rows of a ragged append (one launch takes at most MAX_ITEMS rows).
struct RowSlots {
    uint64_t slot[MAX_ITEMS];
};

// Row r goes to slot slot0 + r, or (RAGGED) to sl.slot[r].
template <typename KVT, bool RAGGED>
__global__ __launch_bounds__(256) void k_rope_append(float* __restrict__ q, const float* __restrict__ k,
                                                     const float* __restrict__ v, KVT* __restrict__ kc,
                                                     KVT* __restrict__ vc, const float* __restrict__ inv_freq,
                                                     const uint32_t* __restrict__ positions, uint32_t rows,
                                                     uint32_t nh, uint32_t nkv, uint32_t hd, uint32_t rope_dim,
                                                     uint32_t neox, uint64_t slot0, const RowSlots sl) {
    const uint32_t half = hd / 2, heads = nh + 2 * nkv;
    const uint64_t idx = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= (uint64_t)rows * heads * half) return;
    const uint32_t p = idx % half, hx = (idx / half) % heads;
    const uint64_t r = idx / ((uint64_t)half * heads);
    const uint64_t kvd = (uint64_t)nkv * hd;
    // Dims of this thread's pair: a rotated pair, or two dims past rope_dim.
    uint32_t a, b;
    const bool rot = rope_pair(p, rope_dim, neox, a, b);
    if (hx < nh) {
        if (!rot) return;
        float* hp = q + (r * nh + hx) * hd;
        const float theta = (float)positions[r] * inv_freq[p];
        float y0, y1;
        rotate(hp[a], hp[b], theta, y0, y1);
        hp[a] = y0;
        hp[b] = y1;
    } else if (hx < nh + nkv) {
        const uint32_t kh = hx - nh;
        const float* hp = k + (r * nkv + kh) * hd;
        float y0 = hp[a], y1 = hp[b];
        if (rot) {
            const float theta = (float)positions[r] * inv_freq[p];
            rotate(hp[a], hp[b], theta, y0, y1);
        }
        KVT* dst = kc + (RAGGED ? sl.slot[r] : slot0 + r) * kvd + (uint64_t)kh * hd;
        dst[a] = to_kv<KVT>(y0);
        dst[b] = to_kv<KVT>(y1);
    } else {
        const uint32_t vh = hx - nh - nkv;
        const float* hp = v + (r * nkv + vh) * hd;
        KVT* dst = vc + (RAGGED ? sl.slot[r] : slot0 + r) * kvd + (uint64_t)vh * hd;
        dst[2 * p] = to_kv<KVT>(hp[2 * p]);
        dst[2 * p + 1] = to_kv<KVT>(hp[2 * p + 1]);
    }
}

static uint32_t blocks_of(uint64_t n) { return (uint32_t)((n + 255) / 256); }

hipError_t rope_launch(float* x, const float* inv_freq, const uint32_t* positions, uint32_t rows,
                       uint32_t heads, uint32_t hd, uint32_t rope_dim, uint32_t neox, hipStream_t s) {
    const uint64_t n = (uint64_t)rows * heads * (rope_dim / 2);
    if (n == 0) return hipSuccess;
    hipLaunchKernelGGL(k_rope, dim3(blocks_of(n)), dim3(256), 0, s, x, inv_freq, positions, rows, heads, hd,
                       rope_dim, neox);
    return hipGetLastError();
}

hipError_t rope_append_launch(float* q, const float* k, const float* v, void* kc, void* vc, uint32_t kv_type,
                              const float* inv_freq, const uint32_t* positions, uint32_t rows, uint32_t nh,
                              uint32_t nkv, uint32_t hd, uint32_t rope_dim, uint32_t neox, uint64_t slot0,
                              hipStream_t s) {
    const uint64_t n = (uint64_t)rows * (nh + 2 * nkv) * (hd / 2);
    if (n == 0) return hipSuccess;
    const RowSlots none{};
    if (kv_type == 1)
        hipLaunchKernelGGL((k_rope_append<f16, false>), dim3(blocks_of(n)), dim3(256), 0, s, q, k, v, (f16*)kc,
                           (f16*)vc, inv_freq, positions, rows, nh, nkv, hd, rope_dim, neox, slot0, none);
    else
        hipLaunchKernelGGL((k_rope_append<float, false>), dim3(blocks_of(n)), dim3(256), 0, s, q, k, v, (float*)kc,
                           (float*)vc, inv_freq, positions, rows, nh, nkv, hd, rope_dim, neox, slot0, none);
    return hipGetLastError();
}

hipError_t rope_append_ragged_launch(float* q, const float* k, const float* v, void* kc, void* vc, uint32_t kv_type,
                                     const float* inv_freq, const uint32_t* positions, uint32_t rows, uint32_t nh,
                                     uint32_t nkv, uint32_t hd, uint32_t rope_dim, uint32_t neox,
                                     const uint64_t* slots, hipStream_t s) {
    for (uint32_t r0 = 0; r0 < rows; r0 += MAX_ITEMS) {
        const uint32_t nr = rows - r0 < MAX_ITEMS ? rows - r0 : MAX_ITEMS;
        RowSlots sl{};
        for (uint32_t i = 0; i < nr; i++) sl.slot[i] = slots[r0 + i];
        const uint64_t n = (uint64_t)nr * (nh + 2 * nkv) * (hd / 2);
        if (n == 0) continue;
        float* qr = q + (size_t)r0 * nh * hd;
        const float* kr = k + (size_t)r0 * nkv * hd;
        const float* vr = v + (size_t)r0 * nkv * hd;
        if (kv_type == 1)
            hipLaunchKernelGGL((k_rope_append<f16, true>), dim3(blocks_of(n)), dim3(256), 0, s, qr, kr, vr, (f16*)kc,
                               (f16*)vc, inv_freq, positions + r0, nr, nh, nkv, hd, rope_dim, neox, 0ull, sl);
        else
            hipLaunchKernelGGL((k_rope_append<float, true>), dim3(blocks_of(n)), dim3(256), 0, s, qr, kr, vr,
                               (float*)kc, (float*)vc, inv_freq, positions + r0, nr, nh, nkv, hd, rope_dim, neox, 0ull,
                               sl);
        hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

}  // namespace bchip
