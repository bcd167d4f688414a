// Shared definitions of the bchip HIP sources: element types, the CDNA4 MFMA tile used by
// every attention kernel, and the launch plans the C ABI hands to the kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace bchip {

typedef _Float16 f16;
typedef f16 half8 __attribute__((ext_vector_type(8)));
typedef f16 half4 __attribute__((ext_vector_type(4)));
typedef f16 half2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

// List entries (visible KV slots) per attention block: four 16-key MFMA tiles.
constexpr int BLK = 64;
// List entries per chunk in every multi-row call. A row's result is the left fold of its
// chunks' (max, sum, weighted values), each chunk an online softmax over its blocks from
// a fresh state, so a chunk may be computed by any workgroup and the row's bits do not
// change: that is what lets a speculative verify split across CUs and still match a
// prefill row exactly.
constexpr uint32_t CHUNK_MULTI = 192;
// Largest head dimension (the reference's MAX_HEAD, kernels.h:31).
constexpr uint32_t MAX_HD = 256;
// Rows a tree pass may hold (model.rs:408), and items one direct launch takes.
constexpr uint32_t MAX_ITEMS = 64;  // at most one a lane: a wave finds a unit's item by one ballot

constexpr float LOG2E = 1.4426950408889634f;

// One 16x16x32 f16 MFMA with f32 accumulate (gfx950). Lane l holds A[l%16][8(l/16)+j],
// B[8(l/16)+j][l%16] (j < 8) and D[4(l/16)+i][l%16] (i < 4).
__device__ __forceinline__ f32x4 mfma16(half8 a, half8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ float exp2_hw(float x) { return __builtin_amdgcn_exp2f(x); }

// Coefficients of merging a softmax state with max M (log2 units) and one with max m: new
// max Mn, weights a (for the first) and b (for the second). An empty state (max -inf) gets
// weight 0 and the other weight exactly 1 (2^0), so folding an empty state in, or folding
// into an empty state, leaves the other exactly as it was. Every fold of chunk states (in a
// kernel or in attn_combine) uses this and the same per-element expression,
// R = R * a + c * b, so a fold gives the same bits wherever it runs.
__device__ __forceinline__ void merge_coef(float M, float m, float& a, float& b, float& Mn) {
    Mn = fmaxf(M, m);
    float ms = (Mn == -INFINITY) ? 0.0f : Mn;
    a = exp2_hw(M - ms);
    b = exp2_hw(m - ms);
}

// Position of the k-th set bit of (lo, hi), k < popcount.
__device__ __forceinline__ uint32_t nth_set_bit(uint32_t lo, uint32_t hi, uint32_t k) {
    uint32_t cl = __popc(lo);
    uint32_t w = k < cl ? lo : hi, off = k < cl ? 0u : 32u;
    k = k < cl ? k : k - cl;
    for (uint32_t i = 0; i < k; i++) w &= w - 1u;  // drop the k lowest set bits
    return off + (uint32_t)__builtin_ctz(w);
}

// The rotation of one RoPE pair by theta: y0 = x0 cos - x1 sin, y1 = x0 sin + x1 cos, each
// product rounded on its own (model.rs:395-400), sincosf the device library's full-range
// one. Every kernel that rotates uses this, so a row rotated anywhere has the same bits.
__device__ __forceinline__ void rotate_sc(float x0, float x1, float s, float c, float& y0, float& y1) {
    y0 = x0 * c - x1 * s;
    y1 = x0 * s + x1 * c;
}
__device__ __forceinline__ void rotate(float x0, float x1, float theta, float& y0, float& y1) {
    float s, c;
    sincosf(theta, &s, &c);
    rotate_sc(x0, x1, s, c, y0, y1);
}

// Dims (a, b) of RoPE pair pp of a head of hd dims: a rotated pair when pp < rope_dim/2
// (neox: (pp, pp + rope_dim/2), else (2pp, 2pp+1)), else two dims past rope_dim, unrotated.
__device__ __forceinline__ bool rope_pair(uint32_t pp, uint32_t rope_dim, uint32_t neox, uint32_t& a, uint32_t& b) {
    const uint32_t hh = rope_dim / 2;
    const bool rot = pp < hh;
    a = rot ? (neox ? pp : 2 * pp) : rope_dim + 2 * (pp - hh);
    b = rot ? (neox ? pp + hh : 2 * pp + 1) : a + 1;
    return rot;
}

// A cache element from f32: f16 rounds to nearest even.
template <typename KVT>
__device__ __forceinline__ KVT to_kv(float v);
template <>
__device__ __forceinline__ f16 to_kv<f16>(float v) {
    return (f16)v;
}
template <>
__device__ __forceinline__ float to_kv<float>(float v) {
    return v;
}

// A row of work for the decode kernel: the G query heads of one row against each KV head.
// Its list is cut into nchunk chunks of `chunk` entries, one unit of work each per KV head.
struct Item {
    uint32_t row;    // row of q / out
    uint32_t len;    // visible list length (tree rows: computed from the mask)
    uint32_t unit0;  // first unit of this item in the launch
    uint32_t nchunk; // chunks of this row's list (an upper bound for tree rows)
    uint32_t chunk;  // list entries per chunk (multiple of BLK)
    uint32_t nrows;  // consecutive line rows in this item (1 for decode and tree rows)
    uint64_t kvoff;  // slot offset of the row's cache (ragged pools), else 0
};


// zero: a device page of zeros that lanes with nothing to read load from.
struct DirectParams {
    const void* zero;
    const float* q;
    const void* kc;
    const void* vc;
    float* out;
    float* part_o;  // [unit][16][HD]: chunk states
    float* part_ml; // [unit][16][2]
    uint32_t nunits;
    const uint32_t* masks; // tree: two words per row
    uint32_t nh, nkv, hd, G;
    uint32_t base;  // tree: first tree slot
    uint32_t tree;
    uint64_t slot_limit; // slots the caches hold (tree slots past it read as absent)
    float sc;       // scale * log2(e)
    // One-row steps fused with RoPE and the K/V append of the new row (fuse != 0): q is
    // unrotated on entry and rotated in registers (qw receives the rotated q, as k_rope
    // leaves it); the new K row (knew, f32, rotated here) and V row (vnew) are written to
    // the caches at the item's last slot and used in place of reading that slot.
    uint32_t fuse;
    float* qw;
    const float* knew;
    const float* vnew;
    const float* inv_freq;
    const uint32_t* positions;  // positions[0]: the rotation's position
    uint32_t rope_dim, neox;
    float* qrot;                // [nh][hd]: the rotated q, staged for attn_row_fold to copy into qw
    // One-row launches: each unit takes a run of chunks and writes the run's state (units
    // and states numbered by run), else a chunk.
    uint32_t runs;
    uint32_t nitems;
    Item items[MAX_ITEMS];
};

// Multi-row line attention: a workgroup takes rb rows x all G heads of one KV head.
struct SharedParams {
    const void* zero;
    const float* q;
    const void* kc;
    const void* vc;
    float* out;
    float* part_o;  // [unit][SL][HD]
    float* part_ml; // [unit][SL][2]
    uint32_t rows, nh, nkv, hd, G;
    uint32_t pos;   // slot of row 0
    float sc;
    const void* vt;    // V^T tiles (prefill kernel), vt_npad keys a dim row
    uint32_t vt_npad;
    uint32_t rb;    // rows per workgroup
    uint32_t nrb;   // row blocks
    uint32_t nchunk;// chunks of the longest list (split launches)
    uint32_t split;
    // Split launches folded in the same launch (group fold): each workgroup publishes its
    // chunk state, waits at its group's arrival counter gcnt[grp * GROUP_STRIDE] for the
    // group's other nchunk - 1 workgroups, then folds one slice of the group's outputs.
    // Null: the states go to attn_combine instead. gerr: the word a wait that runs out sets.
    uint32_t* gcnt;
    uint32_t* gerr;
    uint32_t xmap;  // split launches: blocks 8 apart take one group's chunks (one XCD each)
    uint32_t gspread;  // group fold: take the spread path whatever the XCDs (tests)
    uint32_t gspins;   // group fold: polls a wait may take
    // Multi-row passes fused with RoPE and the K/V append (attn_prefill's FUSE form): q is
    // unrotated on entry and left rotated in qw; row r's new k and v (f32 [rows][nkv][hd])
    // go, k rotated, into the caches at slot pos + r, and the launch takes them from LDS for
    // those slots. positions: the rows' rotation positions.
    const float* knew;
    const float* vnew;
    const float* inv_freq;
    const uint32_t* positions;
    uint32_t rope_dim, neox;
    float* qw;
};

struct CombineParams {
    const void* zero;
    float* out;
    const float* part_o;
    const float* part_ml;
    uint32_t nh, nkv, hd, G;
    uint32_t slots;     // partial slots per unit (16 for decode launches, SL for shared)
    uint32_t slots_out; // workgroups per group: one per output slot
    // decode launches: one group per (item, KV head); shared: one per (KV head, row block)
    uint32_t shared;
    uint32_t rows, rb, nrb, nchunk; // shared launches
    uint32_t ngroups;  // groups in the launch
    uint32_t nitems;
    uint32_t long_fold;  // host: lists of more than CMB_RUN chunks may take attn_combine_long
    // An f32 one-row step fused with RoPE (fuse != 0): the fold leaves each output slot's q
    // head rotated (k_rope_append's expressions), every chunk's workgroup having read it.
    uint32_t fuse, rope_dim, neox;
    float* qw;
    const float* inv_freq;
    const uint32_t* positions;
    Item items[MAX_ITEMS];
};

}  // namespace bchip
