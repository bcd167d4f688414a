// KV-cache movement: bc-infer's k_copy and k_move (crates/bc-infer/src/gpu/kernels.h:332-334,
// entries cuda.cu:89-90), f16-aware, plus Cache::keep for every layer in one launch
// (gpu/mod.rs:322-337), the cache growth of Gpu::reserve for every layer in one launch
// (gpu/mod.rs:404-423), and the seeded N(0,1) generator of the benchmark inputs.
#include "common.hpp"
#include "internal.hpp"

#include <math.h>

#include <type_traits>

namespace bchip {

template <typename S, typename D>
__device__ __forceinline__ D conv(S v) {
    return (D)v;
}

template <typename S, typename D>
__global__ __launch_bounds__(256) void k_copy(const S* __restrict__ src, D* __restrict__ dst, uint64_t off,
                                              uint64_t n) {
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (uint64_t)gridDim.x * blockDim.x)
        dst[off + i] = conv<S, D>(src[i]);
}

// Eight elements a thread when both ends are 16-byte aligned: the loads and stores of a group
// are 16-byte vector accesses (two of them for f32), so a wave moves 1-2 KB an instruction.
template <typename T>
struct Vec8;
template <>
struct Vec8<f16> {
    half8 v;
    __device__ __forceinline__ void load(const f16* p) { v = *(const half8*)p; }
    __device__ __forceinline__ void store(f16* p) const { *(half8*)p = v; }
    __device__ __forceinline__ float get(int j) const { return (float)v[j]; }
    __device__ __forceinline__ void set(int j, float x) { v[j] = (f16)x; }
};
template <>
struct Vec8<float> {
    float4 a, b;
    __device__ __forceinline__ void load(const float* p) {
        a = *(const float4*)p;
        b = *(const float4*)(p + 4);
    }
    __device__ __forceinline__ void store(float* p) const {
        *(float4*)p = a;
        *(float4*)(p + 4) = b;
    }
    __device__ __forceinline__ float get(int j) const {
        return j < 4 ? (j == 0 ? a.x : j == 1 ? a.y : j == 2 ? a.z : a.w) : (j == 4 ? b.x : j == 5 ? b.y : j == 6 ? b.z : b.w);
    }
    __device__ __forceinline__ void set(int j, float x) {
        if (j < 4) (j == 0 ? a.x : j == 1 ? a.y : j == 2 ? a.z : a.w) = x;
        else (j == 4 ? b.x : j == 5 ? b.y : j == 6 ? b.z : b.w) = x;
    }
};

template <typename S, typename D>
__global__ __launch_bounds__(256) void k_copy8(const S* __restrict__ src, D* __restrict__ dst, uint64_t groups) {
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < groups;
         i += (uint64_t)gridDim.x * blockDim.x) {
        Vec8<S> in;
        in.load(src + 8 * i);
        if constexpr (std::is_same<S, D>::value) {
            in.store(dst + 8 * i);
        } else {
            Vec8<D> out;
#pragma unroll
            for (int j = 0; j < 8; j++) out.set(j, in.get(j));  // f32 -> f16 rounds to nearest even
            out.store(dst + 8 * i);
        }
    }
}

// One element per thread; ranges of one launch never overlap (move_launch cuts them).
template <typename T>
__global__ __launch_bounds__(256) void k_move(T* b, uint64_t from, uint64_t to, uint64_t n) {
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (uint64_t)gridDim.x * blockDim.x)
        b[to + i] = b[from + i];
}

struct KeepArgs {
    void* bufs[64];
    uint32_t rows[64];
};

// Each thread owns one element column of one buffer and applies the moves in ascending
// order, as Kv::keep does (model.rs:158-161). Move i reads row base+rows[i] and writes row
// base+i; a later move j > i writes row base+j, which may be a row a move before it read
// (rows[i] = j), so the order matters and is kept per column.
template <typename T>
__global__ __launch_bounds__(256) void k_keep(const KeepArgs a, uint32_t nbufs, uint32_t width, uint64_t base,
                                              uint32_t nrows) {
    const uint32_t col = blockIdx.x * blockDim.x + threadIdx.x;
    const uint32_t bi = blockIdx.y;
    if (col >= width || bi >= nbufs) return;
    T* b = (T*)a.bufs[bi];
    for (uint32_t i = 0; i < nrows; i++) {
        const uint32_t r = a.rows[i];
        if (r != i) b[(base + i) * width + col] = b[(base + r) * width + col];
    }
}

struct GrowArgs {
    const uint8_t* src[64];
    uint8_t* dst[64];
};

// Cache growth for every layer's K and V in one launch: buffer blockIdx.y gets
// dst[0, keep) = src[0, keep) and dst[keep, total) = 0 (bytes), 16 bytes a thread; the one
// 16-byte piece that straddles keep goes byte by byte, so src is never read past keep.
__global__ __launch_bounds__(256) void k_grow(const GrowArgs a, uint64_t keep, uint64_t total) {
    const uint8_t* src = a.src[blockIdx.y];
    uint8_t* dst = a.dst[blockIdx.y];
    const uint64_t pieces = (total + 15) / 16;
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < pieces; i += (uint64_t)gridDim.x * blockDim.x) {
        const uint64_t b0 = 16 * i;
        if (b0 + 16 <= keep) {
            *(uint4*)(dst + b0) = *(const uint4*)(src + b0);
        } else if (b0 >= keep && b0 + 16 <= total) {
            *(uint4*)(dst + b0) = uint4{0u, 0u, 0u, 0u};
        } else {
            for (uint64_t b = b0; b < b0 + 16 && b < total; b++) dst[b] = b < keep ? src[b] : (uint8_t)0;
        }
    }
}

__device__ __forceinline__ uint64_t splitmix64_at(uint64_t seed, uint64_t k) {
    // Output k (from 0) of the sequence whose state starts at seed.
    uint64_t z = seed + (k + 1) * 0x9e3779b97f4a7c15ull;
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
    return z ^ (z >> 31);
}

template <typename T>
__global__ __launch_bounds__(256) void k_fill_normal(T* __restrict__ dst, uint64_t n, uint64_t seed) {
    const double two_pi = 6.283185307179586476925286766559;
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; 2 * i < n;
         i += (uint64_t)gridDim.x * blockDim.x) {
        double u1 = ((double)(splitmix64_at(seed, 2 * i) >> 11) + 1.0) * 0x1.0p-53;
        double u2 = (double)(splitmix64_at(seed, 2 * i + 1) >> 11) * 0x1.0p-53;
        double r = sqrt(-2.0 * log(u1));
        dst[2 * i] = (T)(float)(r * cos(two_pi * u2));
        if (2 * i + 1 < n) dst[2 * i + 1] = (T)(float)(r * sin(two_pi * u2));
    }
}

static uint32_t grid_of(uint64_t n) {
    uint64_t b = (n + 255) / 256;
    return (uint32_t)(b > 65536 ? 65536 : (b ? b : 1));
}

template <typename S, typename D>
static hipError_t copy_t(const S* src, D* dst, uint64_t n, hipStream_t s) {
    uint64_t done = 0;
    if (((uintptr_t)src | (uintptr_t)dst) % 16 == 0 && n >= 8) {
        const uint64_t groups = n / 8;
        hipLaunchKernelGGL((k_copy8<S, D>), dim3(grid_of(groups)), dim3(256), 0, s, src, dst, groups);
        hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
        done = groups * 8;
    }
    if (done < n)
        hipLaunchKernelGGL((k_copy<S, D>), dim3(grid_of(n - done)), dim3(256), 0, s, src + done, dst, done,
                           n - done);
    return hipGetLastError();
}

hipError_t copy_launch(const void* src, uint32_t st, void* dst, uint32_t dt, uint64_t off, uint64_t n, hipStream_t s) {
    if (n == 0) return hipSuccess;
    if (st == 0 && dt == 0) return copy_t((const float*)src, (float*)dst + off, n, s);
    if (st == 0 && dt == 1) return copy_t((const float*)src, (f16*)dst + off, n, s);
    if (st == 1 && dt == 0) return copy_t((const f16*)src, (float*)dst + off, n, s);
    return copy_t((const f16*)src, (f16*)dst + off, n, s);
}

hipError_t move_launch(void* buf, uint32_t type, uint64_t from, uint64_t to, uint64_t n, hipStream_t s) {
    if (n == 0 || from == to) return hipSuccess;
    // With from - to < n the ranges overlap: move in pieces of from - to, in order; each
    // piece's source lies past its destination, and the pieces run one after another.
    const uint64_t step = (from - to < n) ? from - to : n;
    for (uint64_t o = 0; o < n; o += step) {
        const uint64_t m = (n - o < step) ? n - o : step;
        if (type == 1)
            hipLaunchKernelGGL(k_move<f16>, dim3(grid_of(m)), dim3(256), 0, s, (f16*)buf, from + o, to + o, m);
        else
            hipLaunchKernelGGL(k_move<float>, dim3(grid_of(m)), dim3(256), 0, s, (float*)buf, from + o, to + o, m);
        hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

hipError_t keep_launch(void* const* bufs, uint32_t nbufs, uint32_t type, uint32_t width, uint64_t base,
                       const uint32_t* rows, uint32_t nrows, hipStream_t s) {
    if (nbufs == 0 || nrows == 0 || width == 0) return hipSuccess;
    for (uint32_t b0 = 0; b0 < nbufs; b0 += 64) {
        KeepArgs a{};
        const uint32_t nb = (nbufs - b0 < 64) ? nbufs - b0 : 64;
        for (uint32_t i = 0; i < nb; i++) a.bufs[i] = bufs[b0 + i];
        for (uint32_t i = 0; i < nrows; i++) a.rows[i] = rows[i];
        dim3 g((width + 255) / 256, nb);
        if (type == 1)
            hipLaunchKernelGGL(k_keep<f16>, g, dim3(256), 0, s, a, nb, width, base, nrows);
        else
            hipLaunchKernelGGL(k_keep<float>, g, dim3(256), 0, s, a, nb, width, base, nrows);
        hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

hipError_t grow_launch(const void* const* src, void* const* dst, uint32_t nbufs, uint64_t keep_bytes,
                       uint64_t total_bytes, hipStream_t s) {
    if (nbufs == 0 || total_bytes == 0) return hipSuccess;
    for (uint32_t b0 = 0; b0 < nbufs; b0 += 64) {
        GrowArgs a{};
        const uint32_t nb = (nbufs - b0 < 64) ? nbufs - b0 : 64;
        for (uint32_t i = 0; i < nb; i++) {
            a.src[i] = (const uint8_t*)src[b0 + i];
            a.dst[i] = (uint8_t*)dst[b0 + i];
        }
        const uint64_t pieces = (total_bytes + 15) / 16;
        const uint32_t gx = (uint32_t)((pieces + 255) / 256 > 2048 ? 2048 : (pieces + 255) / 256);
        hipLaunchKernelGGL(k_grow, dim3(gx, nb), dim3(256), 0, s, a, keep_bytes, total_bytes);
        hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

hipError_t fill_normal_launch(void* dst, uint32_t type, uint64_t n, uint64_t seed, hipStream_t s) {
    if (n == 0) return hipSuccess;
    const uint64_t pairs = (n + 1) / 2;
    if (type == 1)
        hipLaunchKernelGGL(k_fill_normal<f16>, dim3(grid_of(pairs)), dim3(256), 0, s, (f16*)dst, n, seed);
    else
        hipLaunchKernelGGL(k_fill_normal<float>, dim3(grid_of(pairs)), dim3(256), 0, s, (float*)dst, n, seed);
    return hipGetLastError();
}

}  // namespace bchip
