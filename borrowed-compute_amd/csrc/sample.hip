// The next-token pick on the device: bc-infer's sampler (crates/bc-infer/src/sample.rs:24-71),
// the step after the logits head (gpu/mod.rs:499-508), with the reference's results index for
// index.
//
// Temperature 0: the first index of the highest score (sample.rs:24-32), a parallel argmax
// whose ties go to the lower index. Otherwise, per row (sample.rs:35-71):
//   max = the largest non-NaN score; p_i = exp((s_i - max) / T) with exp correctly rounded
//     (computed in double, as the CPU restatement does; the reference leaves exp to libm);
//   total = sum of p_i in index order, from -0: one lane adds them in that order (a parallel
//     sum would round differently);
//   the stable descending sort by f32::total_cmp: a stable radix sort (rocPRIM) of 64-bit keys,
//     the p key of the total order inverted over the index;
//   keep = the shortest sorted prefix whose running mass (sum of p / total, each step
//     rounded) reaches top_p, at least 1; r = uniform(seed ^ step * golden) * (sum of the kept
//     p, in order); the first kept token whose running r -= p reaches <= 0, else the first.
// The sequential loops read the sorted keys through LDS, staged by the whole workgroup.
#include <cstring>  // before rocPRIM, whose iterator header calls memset

#include <rocprim/device/device_radix_sort.hpp>

#include "common.hpp"
#include "internal.hpp"

#include <math.h>

namespace bchip {

constexpr int SMP_THREADS = 1024;
constexpr uint32_t SMP_CHUNK = 8192;  // LDS staging of the sequential loops (64 KB of keys)

// f32::total_cmp as an unsigned key: ascending keys are ascending total order.
__device__ __forceinline__ uint32_t total_key(float x) {
    const uint32_t b = __float_as_uint(x);
    return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}
__device__ __forceinline__ float from_total_key(uint32_t k) {
    return __uint_as_float((k & 0x80000000u) ? (k & 0x7fffffffu) : ~k);
}

// Sort key of token i: descending total order of its p, then ascending index (the stable sort).
__device__ __forceinline__ uint64_t sort_key(float p, uint32_t i) {
    return ((uint64_t)(~total_key(p)) << 32) | i;
}
__device__ __forceinline__ float key_weight(uint64_t k) { return from_total_key(~(uint32_t)(k >> 32)); }

// sample.rs:74-81.
__device__ __forceinline__ float uniform(uint64_t seed) {
    uint64_t z = seed + 0x9e3779b97f4a7c15ull;
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
    z ^= z >> 31;
    return (float)(z >> 40) / (float)(1ull << 24);
}

// The highest score of a row and its first index: the reference's argmax starts from index 0
// and moves only on a strictly higher score, so a NaN never wins past index 0, and a row whose
// first score is NaN answers 0.
__global__ __launch_bounds__(SMP_THREADS) void k_argmax(const float* __restrict__ scores, uint32_t vocab,
                                                        uint32_t* __restrict__ ids) {
    __shared__ float bv_s[SMP_THREADS / 64];
    __shared__ uint32_t bi_s[SMP_THREADS / 64];
    const float* s = scores + (size_t)blockIdx.x * vocab;
    const uint32_t tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    float bv = -INFINITY;
    uint32_t bi = 0xffffffffu;
    for (uint32_t i = tid; i < vocab; i += SMP_THREADS) {
        const float v = s[i];
        if (v > bv) {  // strict: the first occurrence in this thread's ascending indices
            bv = v;
            bi = i;
        }
    }
    auto better = [](float v, uint32_t i, float bv, uint32_t bi) { return v > bv || (v == bv && i < bi); };
#pragma unroll
    for (int d = 1; d < 64; d *= 2) {
        const float ov = __shfl_xor(bv, d);
        const uint32_t oi = __shfl_xor(bi, d);
        if (better(ov, oi, bv, bi)) {
            bv = ov;
            bi = oi;
        }
    }
    if (lane == 0) {
        bv_s[w] = bv;
        bi_s[w] = bi;
    }
    __syncthreads();
    if (tid == 0) {
        for (int j = 1; j < SMP_THREADS / 64; j++)
            if (better(bv_s[j], bi_s[j], bv, bi)) {
                bv = bv_s[j];
                bi = bi_s[j];
            }
        // No score above -inf (or only NaN past index 0), or a NaN at index 0: index 0.
        ids[blockIdx.x] = (bi == 0xffffffffu || isnan(s[0])) ? 0u : bi;
    }
}

// Per row: the max, p_i and their sort keys, and total (one lane, index order).
__global__ __launch_bounds__(SMP_THREADS) void k_sample_prep(const float* __restrict__ scores, uint32_t vocab,
                                                             float temperature, uint64_t* __restrict__ keys,
                                                             float* __restrict__ totals) {
    __shared__ float red[SMP_THREADS / 64];
    __shared__ float stage[SMP_CHUNK];
    const uint32_t tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const float* s = scores + (size_t)blockIdx.x * vocab;
    uint64_t* kr = keys + (size_t)blockIdx.x * vocab;
    float mx = -INFINITY;
    for (uint32_t i = tid; i < vocab; i += SMP_THREADS) mx = fmaxf(mx, s[i]);  // f32::max skips NaN
#pragma unroll
    for (int d = 1; d < 64; d *= 2) mx = fmaxf(mx, __shfl_xor(mx, d));
    if (lane == 0) red[w] = mx;
    __syncthreads();
    mx = red[0];
    for (int j = 1; j < SMP_THREADS / 64; j++) mx = fmaxf(mx, red[j]);
    float total = -0.0f;  // Iterator::sum over f32
    for (uint32_t c0 = 0; c0 < vocab; c0 += SMP_CHUNK) {
        const uint32_t n = min(SMP_CHUNK, vocab - c0);
        for (uint32_t j = tid; j < n; j += SMP_THREADS) {
            const float p = (float)exp((double)((s[c0 + j] - mx) / temperature));
            stage[j] = p;
            kr[c0 + j] = sort_key(p, c0 + j);
        }
        __syncthreads();
        if (tid == 0)
            for (uint32_t j = 0; j < n; j++) total += stage[j];
        __syncthreads();
    }
    if (tid == 0) totals[blockIdx.x] = total;
}

// Per row: the nucleus and the draw over the sorted keys (one lane, sorted order).
__global__ __launch_bounds__(SMP_THREADS) void k_sample_draw(const uint64_t* __restrict__ sorted, uint32_t vocab,
                                                             const float* __restrict__ totals, float top_p,
                                                             uint64_t seed, uint64_t step0,
                                                             uint32_t* __restrict__ ids) {
    __shared__ uint64_t stage[SMP_CHUNK];
    __shared__ uint32_t flag;
    const uint32_t tid = threadIdx.x, row = blockIdx.x;
    const uint64_t* kr = sorted + (size_t)row * vocab;
    const float total = totals[row];
    // Pass 1: keep (the running mass reaches top_p).
    uint32_t keep = 0;
    float mass = 0.0f;
    if (tid == 0) flag = 0;
    for (uint32_t c0 = 0; c0 < vocab; c0 += SMP_CHUNK) {
        const uint32_t n = min(SMP_CHUNK, vocab - c0);
        __syncthreads();
        if (flag) break;
        for (uint32_t j = tid; j < n; j += SMP_THREADS) stage[j] = kr[c0 + j];
        __syncthreads();
        if (tid == 0) {
            for (uint32_t j = 0; j < n; j++) {
                keep++;
                mass += key_weight(stage[j]) / total;
                if (mass >= top_p) {
                    flag = 1;
                    break;
                }
            }
        }
    }
    __syncthreads();
    __shared__ uint32_t keep_s;
    if (tid == 0) keep_s = keep < 1 ? 1u : keep;
    __syncthreads();
    keep = keep_s;
    // Pass 2: the kept mass, in sorted order from -0.
    float kept = -0.0f;
    for (uint32_t c0 = 0; c0 < keep; c0 += SMP_CHUNK) {
        const uint32_t n = min(SMP_CHUNK, keep - c0);
        __syncthreads();
        for (uint32_t j = tid; j < n; j += SMP_THREADS) stage[j] = kr[c0 + j];
        __syncthreads();
        if (tid == 0)
            for (uint32_t j = 0; j < n; j++) kept += key_weight(stage[j]);
    }
    // Pass 3: the draw.
    const uint64_t step = step0 + row;
    float r = uniform(seed ^ (step * 0x9e3779b97f4a7c15ull)) * kept;
    uint32_t id = (uint32_t)(kr[0] & 0xffffffffu);
    if (tid == 0) flag = 0;
    for (uint32_t c0 = 0; c0 < keep; c0 += SMP_CHUNK) {
        const uint32_t n = min(SMP_CHUNK, keep - c0);
        __syncthreads();
        if (flag) break;
        for (uint32_t j = tid; j < n; j += SMP_THREADS) stage[j] = kr[c0 + j];
        __syncthreads();
        if (tid == 0) {
            for (uint32_t j = 0; j < n; j++) {
                r -= key_weight(stage[j]);
                if (r <= 0.0f) {
                    id = (uint32_t)(stage[j] & 0xffffffffu);
                    flag = 1;
                    break;
                }
            }
        }
    }
    if (tid == 0) ids[row] = id;
}

size_t sample_scratch_bytes(uint32_t rows, uint32_t vocab) {
    size_t sort_bytes = 0;
    (void)rocprim::radix_sort_keys(nullptr, sort_bytes, (const uint64_t*)nullptr, (uint64_t*)nullptr, vocab, 0, 64);
    const size_t keys = (size_t)rows * vocab * sizeof(uint64_t);
    return 2 * keys + (size_t)rows * sizeof(float) + ((sort_bytes + 255) & ~(size_t)255) + 1024;
}

hipError_t sample_launch(const float* scores, uint32_t rows, uint32_t vocab, float temperature, float top_p,
                         uint64_t seed, uint64_t step0, uint32_t* ids, void* scratch, size_t scratch_bytes,
                         hipStream_t s) {
    if (rows == 0 || vocab == 0) return hipSuccess;
    if (!(temperature > 0.0f)) {
        hipLaunchKernelGGL(k_argmax, dim3(rows), dim3(SMP_THREADS), 0, s, scores, vocab, ids);
        return hipGetLastError();
    }
    size_t sort_bytes = 0;
    hipError_t e = rocprim::radix_sort_keys(nullptr, sort_bytes, (const uint64_t*)nullptr, (uint64_t*)nullptr, vocab,
                                            0, 64, s);
    if (e != hipSuccess) return e;
    const size_t keys = (size_t)rows * vocab * sizeof(uint64_t);
    char* base = (char*)(((uintptr_t)scratch + 255) & ~(uintptr_t)255);
    uint64_t* kin = (uint64_t*)base;
    uint64_t* kout = (uint64_t*)(base + keys);
    float* totals = (float*)(base + 2 * keys);
    void* tmp = (void*)(((uintptr_t)(totals + rows) + 255) & ~(uintptr_t)255);
    if ((char*)tmp + sort_bytes > (char*)scratch + scratch_bytes) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_sample_prep, dim3(rows), dim3(SMP_THREADS), 0, s, scores, vocab, temperature, kin, totals);
    e = hipGetLastError();
    if (e != hipSuccess) return e;
    for (uint32_t r = 0; r < rows; r++) {
        size_t b = sort_bytes;
        e = rocprim::radix_sort_keys(tmp, b, kin + (size_t)r * vocab, kout + (size_t)r * vocab, vocab, 0, 64, s);
        if (e != hipSuccess) return e;
    }
    hipLaunchKernelGGL(k_sample_draw, dim3(rows), dim3(SMP_THREADS), 0, s, kout, vocab, totals, top_p, seed, step0,
                       ids);
    return hipGetLastError();
}

}  // namespace bchip
