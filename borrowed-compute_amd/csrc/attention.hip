// Causal grouped-query attention on CDNA4 MFMA tiles: bc-infer's k_attention
// (crates/bc-infer/src/gpu/kernels.h:250-324, entry cuda.cu:82-85) re-designed for gfx950.
//
// What the reference does, per (row, head): an online softmax over 1024-slot tiles,
// one K row per lane read serially over head_dim, the KV head re-read by every query
// head of its group, 32 threads a head, no split over the KV length.
//
// What this does: a 16-slot MFMA tile holds query slots (row, head) that share one KV
// head. Per block of 64 visible list entries:
//   S^T[key][slot] = K . Q^T        4 key tiles x hd/32 MFMAs 16x16x32 f16 (f32 accumulate)
//   online softmax in log2 units    per slot: running max m, sum l (of the f16-rounded p)
//   O^T[hd][slot] += V^T . P^T      hd/16 x 2 MFMAs; P^T comes straight out of S^T's
//                                   registers (the key order inside the MFMA k-dimension is
//                                   chosen so), V^T is V transposed through LDS.
// A row's list is cut into chunks; each chunk is an online softmax from a fresh state and
// the row's result is the left fold of its chunks' (m, l, O) (merge below). The same code
// computes every chunk, whichever workgroup runs it, so a chunk can run on any CU:
//  - attn_direct: one wave, one tile = the G heads of one row; K straight from HBM into
//    MFMA operands, V through a per-wave LDS tile. One-row decode (split across CUs by
//    chunk), ragged multi-sequence decode, and tree rows (each row gathers its own list).
//  - attn_shared: four waves share K/V blocks staged in LDS (double-buffered) for up to
//    128 slots (rows x G heads of one KV head): prefill and line verify.
//  - attn_combine: the left fold of split chunks, in chunk order.
// Every product of the fold, the softmax and the normalisation rounds on its own (the
// library is built with -ffp-contract=off), so the fold is the same bits in a register
// loop and in attn_combine.
#include "common.hpp"
#include "internal.hpp"

#include <math.h>

namespace bchip {

// f16 per row of the transposed V tile in LDS: 64 keys + 4 pad (8-byte aligned rows).
constexpr int VTS = BLK + 4;

template <int HD>
struct State {
    f32x4 o[HD / 16];  // O^T[16*dt + 4*(lane/16) + i][lane%16]
    float m, l;        // running max (log2 units) and sum of this lane's slot
};

template <int HD>
__device__ __forceinline__ void state_clear(State<HD>& s) {
#pragma unroll
    for (int i = 0; i < HD / 16; i++) s.o[i] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    s.m = -INFINITY;
    s.l = 0.0f;
}

__device__ __forceinline__ float exp2_hw(float x) { return __builtin_amdgcn_exp2f(x); }

// Coefficients of merging a state with max M and one with max m: new max Mn, weights a
// (for the first) and b (for the second). An empty state (max -inf) gets weight 0, and
// merging into an empty state leaves the other exactly as it was.
__device__ __forceinline__ void merge_coef(float M, float m, float& a, float& b, float& Mn) {
    Mn = fmaxf(M, m);
    float ms = (Mn == -INFINITY) ? 0.0f : Mn;
    a = exp2_hw(M - ms);
    b = exp2_hw(m - ms);
}

// R <- fold(R, c). The per-element expression is the one attn_combine uses.
template <int HD>
__device__ __forceinline__ void fold(State<HD>& R, const State<HD>& c) {
    float a, b, mn;
    merge_coef(R.m, c.m, a, b, mn);
    R.l = R.l * a + c.l * b;
#pragma unroll
    for (int i = 0; i < HD / 16; i++) R.o[i] = R.o[i] * a + c.o[i] * b;
    R.m = mn;
}

// The V^T operand of one PV MFMA: lane (g, n) holds V[key(g, j)][16*dt + n] for the
// k-dimension order key(g, j) = 32*kc + 16*(j/4) + 4*g + j%4, the order in which this
// lane holds P^T after the score MFMAs.
__device__ __forceinline__ half8 v_operand(const f16* __restrict__ vt, int dt, int kc, int g, int n) {
    const f16* row = vt + (16 * dt + n) * VTS + 32 * kc + 4 * g;
    half4 a = *(const half4*)row;
    half4 b = *(const half4*)(row + 16);
    return half8{a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]};
}

// One block of 64 list entries [key0, key0+64) for NT tiles of one wave.
// kop(kt, c) gives the K operand of key tile kt (keys key0+16kt..) and hd chunk c:
// lane (g, n) holds K[key0 + 16kt + n][32c + 8g .. +8]. vt is V^T of the block in LDS.
// len[t] is the list length of this lane's slot in tile t (entries >= len are masked).
template <int HD, int NT, typename KOp>
__device__ __forceinline__ void block_step(State<HD> (&s)[NT], const half8 (&qb)[NT][HD / 32], KOp kop,
                                           const f16* __restrict__ vt, uint32_t key0,
                                           const uint32_t (&len)[NT], float sc) {
    const int lane = threadIdx.x & 63;
    const int g = lane >> 4, n = lane & 15;
    f32x4 st[NT][4];
#pragma unroll
    for (int kt = 0; kt < 4; kt++) {
#pragma unroll
        for (int t = 0; t < NT; t++) st[t][kt] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int c = 0; c < HD / 32; c++) {
            half8 a = kop(kt, c);
#pragma unroll
            for (int t = 0; t < NT; t++) st[t][kt] = mfma16(a, qb[t][c], st[t][kt]);
        }
    }
    half8 pb[NT][2];
#pragma unroll
    for (int t = 0; t < NT; t++) {
        float mx = -INFINITY;
        float x[4][4];
#pragma unroll
        for (int kt = 0; kt < 4; kt++)
#pragma unroll
            for (int i = 0; i < 4; i++) {
                uint32_t k = key0 + 16 * kt + 4 * g + i;
                float v = st[t][kt][i] * sc;
                x[kt][i] = (k < len[t]) ? v : -INFINITY;
                mx = fmaxf(mx, x[kt][i]);
            }
        mx = fmaxf(mx, __shfl_xor(mx, 16));
        mx = fmaxf(mx, __shfl_xor(mx, 32));
        float mn = fmaxf(s[t].m, mx);
        float ms = (mn == -INFINITY) ? 0.0f : mn;
        float corr = exp2_hw(s[t].m - ms);
        float ps = 0.0f;
#pragma unroll
        for (int kt = 0; kt < 4; kt++)
#pragma unroll
            for (int i = 0; i < 4; i++) {
                f16 ph = (f16)exp2_hw(x[kt][i] - ms);
                ps = ps + (float)ph;
                pb[t][kt >> 1][(kt & 1) * 4 + i] = ph;
            }
        ps = ps + __shfl_xor(ps, 16);
        ps = ps + __shfl_xor(ps, 32);
        s[t].l = s[t].l * corr + ps;
        s[t].m = mn;
#pragma unroll
        for (int dt = 0; dt < HD / 16; dt++) s[t].o[dt] = s[t].o[dt] * corr;
    }
#pragma unroll
    for (int dt = 0; dt < HD / 16; dt++)
#pragma unroll
        for (int kc = 0; kc < 2; kc++) {
            half8 a = v_operand(vt, dt, kc, g, n);
#pragma unroll
            for (int t = 0; t < NT; t++) s[t].o[dt] = mfma16(a, pb[t][kc], s[t].o[dt]);
        }
}

// 8 consecutive elements of a cache row as f16 (f32 caches are rounded to nearest even).
template <typename KVT>
__device__ __forceinline__ half8 load8(const KVT* p);
template <>
__device__ __forceinline__ half8 load8<f16>(const f16* p) {
    return *(const half8*)p;
}
template <>
__device__ __forceinline__ half8 load8<float>(const float* p) {
    float4 a = *(const float4*)p, b = *(const float4*)(p + 4);
    return half8{(f16)a.x, (f16)a.y, (f16)a.z, (f16)a.w, (f16)b.x, (f16)b.y, (f16)b.z, (f16)b.w};
}

__device__ __forceinline__ half8 q_operand(const float* __restrict__ qrow, uint32_t hd0, uint32_t hd, bool ok) {
    if (!ok || hd0 >= hd) return half8{0, 0, 0, 0, 0, 0, 0, 0};
    float4 a = *(const float4*)(qrow + hd0), b = *(const float4*)(qrow + hd0 + 4);
    return half8{(f16)a.x, (f16)a.y, (f16)a.z, (f16)a.w, (f16)b.x, (f16)b.y, (f16)b.z, (f16)b.w};
}

// Writes the 8 f16 values of key kl, dims hd0..hd0+7, into the transposed tile vt.
__device__ __forceinline__ void vt_store(f16* __restrict__ vt, int kl, uint32_t hd0, half8 v) {
#pragma unroll
    for (int j = 0; j < 8; j++) vt[(hd0 + j) * VTS + kl] = v[j];
}

// Position of the k-th set bit of (lo, hi), k < popcount.
__device__ __forceinline__ uint32_t nth_set_bit(uint32_t lo, uint32_t hi, uint32_t k) {
    uint32_t cl = __popc(lo);
    uint32_t w = k < cl ? lo : hi, off = k < cl ? 0u : 32u;
    k = k < cl ? k : k - cl;
    for (uint32_t i = 0; i < k; i++) w &= w - 1u;  // drop the k lowest set bits
    return off + (uint32_t)__builtin_ctz(w);
}

// ---------------------------------------------------------------------------------------
// Direct kernel: one wave = one row's G heads x one KV head x (one chunk | all chunks).
template <int HD, typename KVT>
__global__ __launch_bounds__(64) void attn_direct(const DirectParams p) {
    __shared__ __attribute__((aligned(16))) f16 vt[HD * VTS];
    __shared__ uint32_t tail[64];
    const int lane = threadIdx.x;
    const int g = lane >> 4, n = lane & 15;
    const uint32_t u = blockIdx.x;
    const uint32_t per = p.split ? 0u : 1u;
    uint32_t it = 0;
    for (; it + 1 < p.nitems; it++) {
        const Item& I = p.items[it];
        if (u < I.unit0 + p.nkv * (per ? 1u : I.nchunk)) break;
    }
    const Item I = p.items[it];
    const uint32_t rem = u - I.unit0;
    uint32_t kvh, c0, c1;
    if (p.split) {
        kvh = rem / I.nchunk;
        c0 = rem % I.nchunk;
        c1 = c0 + 1;
    } else {
        kvh = rem;
        c0 = 0;
        c1 = I.nchunk;
    }
    uint32_t len = I.len;
    if (p.tree) {
        const uint32_t lo = p.masks[2 * I.row], hi = p.masks[2 * I.row + 1];
        const uint32_t ntail = __popc(lo) + __popc(hi);
        len = p.base + ntail;
        if ((uint32_t)lane < ntail) tail[lane] = p.base + nth_set_bit(lo, hi, lane);
        __syncthreads();
    }
    const uint32_t hd = p.hd, kvd = p.nkv * hd;
    const bool valid = (uint32_t)n < p.G;
    const uint32_t h = kvh * p.G + n;
    half8 qb[1][HD / 32];
    {
        const float* qrow = p.q + ((size_t)I.row * p.nh + (valid ? h : 0u)) * hd;
#pragma unroll
        for (int c = 0; c < HD / 32; c++) qb[0][c] = q_operand(qrow, 32 * c + 8 * g, hd, valid);
    }
    const KVT* kc = (const KVT*)p.kc + I.kvoff * kvd + (size_t)kvh * hd;
    const KVT* vc = (const KVT*)p.vc + I.kvoff * kvd + (size_t)kvh * hd;
    // Cache slot of list entry k, or ok = false for entries past the list (and for tree
    // slots past the cache, which a bad mask could name): those read as zeros.
    auto slot_of = [&](uint32_t k, bool& ok) -> uint32_t {
        ok = k < len;
        if (!ok) return 0u;
        const uint32_t s = (!p.tree || k < p.base) ? k : tail[k - p.base];
        ok = (uint64_t)s + I.kvoff < p.slot_limit;
        return ok ? s : 0u;
    };
    const uint32_t lens[1] = {len};
    State<HD> R[1];
    state_clear(R[0]);
    constexpr int LPR = HD / 8;       // lanes per V row (16 bytes each)
    constexpr int KPI = 64 / LPR;     // V rows per load
    for (uint32_t cc = c0; cc < c1; cc++) {
        State<HD> cs[1];
        state_clear(cs[0]);
        const uint32_t kbeg = cc * I.chunk;
        const uint32_t kend = min(kbeg + I.chunk, len);
        for (uint32_t key0 = kbeg; key0 < kend; key0 += BLK) {
            half8 kreg[4][HD / 32];
#pragma unroll
            for (int kt = 0; kt < 4; kt++) {
                bool ok;
                const KVT* row = kc + (size_t)slot_of(key0 + 16 * kt + n, ok) * kvd;
#pragma unroll
                for (int c = 0; c < HD / 32; c++) {
                    uint32_t hd0 = 32 * c + 8 * g;
                    kreg[kt][c] = (ok && hd0 < hd) ? load8<KVT>(row + hd0) : half8{0, 0, 0, 0, 0, 0, 0, 0};
                }
            }
#pragma unroll
            for (int i = 0; i < BLK / KPI; i++) {
                int kl = i * KPI + lane / LPR;
                uint32_t hd0 = 8 * (lane % LPR);
                bool ok;
                const KVT* row = vc + (size_t)slot_of(key0 + kl, ok) * kvd;
                half8 v = (ok && hd0 < hd) ? load8<KVT>(row + hd0) : half8{0, 0, 0, 0, 0, 0, 0, 0};
                vt_store(vt, kl, hd0, v);
            }
            __syncthreads();
            block_step<HD, 1>(cs, qb, [&](int kt, int c) { return kreg[kt][c]; }, vt, key0, lens, p.sc);
            __syncthreads();
        }
        if (p.split) {
            float* po = p.part_o + ((size_t)u * 16 + n) * HD;
#pragma unroll
            for (int dt = 0; dt < HD / 16; dt++) {
                uint32_t d = 16 * dt + 4 * g;
                if (d < hd) *(float4*)(po + d) = float4{cs[0].o[dt][0], cs[0].o[dt][1], cs[0].o[dt][2], cs[0].o[dt][3]};
            }
            if (g == 0) *(float2*)(p.part_ml + ((size_t)u * 16 + n) * 2) = float2{cs[0].m, cs[0].l};
        } else {
            fold(R[0], cs[0]);
        }
    }
    if (!p.split && valid) {
        float* orow = p.out + ((size_t)I.row * p.nh + h) * hd;
#pragma unroll
        for (int dt = 0; dt < HD / 16; dt++) {
            uint32_t d = 16 * dt + 4 * g;
            if (d < hd)
                *(float4*)(orow + d) = float4{R[0].o[dt][0] / R[0].l, R[0].o[dt][1] / R[0].l, R[0].o[dt][2] / R[0].l,
                                              R[0].o[dt][3] / R[0].l};
        }
    }
}

// ---------------------------------------------------------------------------------------
// Shared kernel: W waves x NT tiles = up to W*NT*16 slots = rb rows x G heads of one KV
// head; K and V blocks staged once in LDS for all of them, double-buffered.
template <int HD, typename KVT, int W, int NT>
__global__ __launch_bounds__(64 * W) void attn_shared(const SharedParams p) {
    constexpr int SL = W * NT * 16;
    constexpr int KS = HD + 8;          // f16 per K row in LDS
    constexpr int LPR = HD / 8;         // threads per row load (16 bytes each)
    constexpr int NTH = 64 * W;
    constexpr int LOADS = BLK * LPR / NTH;  // row loads per thread per block (K and V each)
    static_assert(BLK * LPR % NTH == 0, "block loads must divide over the threads");
    __shared__ __attribute__((aligned(16))) f16 kl[2][BLK * KS];
    __shared__ __attribute__((aligned(16))) f16 vt[2][HD * VTS];

    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int g = lane >> 4, n = lane & 15;
    // Heaviest row blocks (latest rows, longest lists) first, across KV heads.
    const uint32_t ngrp = p.nkv * p.nrb;
    const uint32_t gi_launch = p.split ? blockIdx.x / p.nchunk : blockIdx.x;
    const uint32_t cs_idx = p.split ? blockIdx.x % p.nchunk : 0u;
    const uint32_t kvh = gi_launch % p.nkv;
    const uint32_t rbi = p.nrb - 1u - gi_launch / p.nkv;
    const uint32_t grp = kvh * p.nrb + rbi;  // canonical group of the partials
    (void)ngrp;
    const uint32_t r0 = rbi * p.rb;
    const uint32_t rlast = min(r0 + p.rb, p.rows) - 1u;
    const uint32_t maxlen = p.pos + rlast + 1u;
    const uint32_t hd = p.hd, kvd = p.nkv * hd;

    half8 qb[NT][HD / 32];
    uint32_t len[NT];
    uint32_t orow[NT], ohead[NT];
    bool valid[NT];
#pragma unroll
    for (int t = 0; t < NT; t++) {
        uint32_t sl = (w * NT + t) * 16 + n;
        uint32_t gh = sl / p.rb, rl = sl % p.rb, r = r0 + rl;
        valid[t] = gh < p.G && r < p.rows;
        len[t] = valid[t] ? p.pos + r + 1u : 0u;
        orow[t] = r;
        ohead[t] = kvh * p.G + gh;
        const float* qrow = p.q + ((size_t)(valid[t] ? r : 0u) * p.nh + (valid[t] ? ohead[t] : 0u)) * hd;
#pragma unroll
        for (int c = 0; c < HD / 32; c++) qb[t][c] = q_operand(qrow, 32 * c + 8 * g, hd, valid[t]);
    }

    const KVT* kcb = (const KVT*)p.kc + (size_t)kvh * hd;
    const KVT* vcb = (const KVT*)p.vc + (size_t)kvh * hd;
    uint32_t kb0, kb1;  // list range of this workgroup
    if (p.split) {
        kb0 = cs_idx * CHUNK_MULTI;
        kb1 = min(kb0 + CHUNK_MULTI, maxlen);
    } else {
        kb0 = 0;
        kb1 = maxlen;
    }

    half8 kpre[LOADS], vpre[LOADS];
    auto load_block = [&](uint32_t key0) {
#pragma unroll
        for (int i = 0; i < LOADS; i++) {
            int e = i * NTH + tid;
            int kr = e / LPR;
            uint32_t hd0 = 8 * (e % LPR);
            uint32_t k = key0 + kr;
            bool ok = k < maxlen && hd0 < hd;
            kpre[i] = ok ? load8<KVT>(kcb + (size_t)k * kvd + hd0) : half8{0, 0, 0, 0, 0, 0, 0, 0};
            vpre[i] = ok ? load8<KVT>(vcb + (size_t)k * kvd + hd0) : half8{0, 0, 0, 0, 0, 0, 0, 0};
        }
    };
    auto store_block = [&](int stage) {
#pragma unroll
        for (int i = 0; i < LOADS; i++) {
            int e = i * NTH + tid;
            int kr = e / LPR;
            uint32_t hd0 = 8 * (e % LPR);
            *(half8*)&kl[stage][kr * KS + hd0] = kpre[i];
            vt_store(vt[stage], kr, hd0, vpre[i]);
        }
    };

    State<HD> R[NT], cs[NT];
#pragma unroll
    for (int t = 0; t < NT; t++) {
        state_clear(R[t]);
        state_clear(cs[t]);
    }
    int stage = 0;
    if (kb0 < kb1) {
        load_block(kb0);
        store_block(0);
    }
    __syncthreads();
    for (uint32_t key0 = kb0; key0 < kb1; key0 += BLK) {
        if (key0 != kb0 && key0 % CHUNK_MULTI == 0) {
#pragma unroll
            for (int t = 0; t < NT; t++) {
                fold(R[t], cs[t]);
                state_clear(cs[t]);
            }
        }
        const bool more = key0 + BLK < kb1;
        if (more) load_block(key0 + BLK);
        const f16* kls = kl[stage];
        block_step<HD, NT>(
            cs, qb,
            [&](int kt, int c) { return *(const half8*)&kls[(16 * kt + n) * KS + 32 * c + 8 * g]; },
            vt[stage], key0, len, p.sc);
        if (more) store_block(stage ^ 1);
        __syncthreads();
        stage ^= 1;
    }
    if (p.split) {
        const size_t u = (size_t)grp * p.nchunk + cs_idx;
#pragma unroll
        for (int t = 0; t < NT; t++) {
            uint32_t sl = (w * NT + t) * 16 + n;
            float* po = p.part_o + (u * SL + sl) * HD;
#pragma unroll
            for (int dt = 0; dt < HD / 16; dt++) {
                uint32_t d = 16 * dt + 4 * g;
                if (d < hd) *(float4*)(po + d) = float4{cs[t].o[dt][0], cs[t].o[dt][1], cs[t].o[dt][2], cs[t].o[dt][3]};
            }
            if (g == 0) *(float2*)(p.part_ml + (u * SL + sl) * 2) = float2{cs[t].m, cs[t].l};
        }
        return;
    }
#pragma unroll
    for (int t = 0; t < NT; t++) {
        fold(R[t], cs[t]);
        if (!valid[t]) continue;
        float* o = p.out + ((size_t)orow[t] * p.nh + ohead[t]) * hd;
#pragma unroll
        for (int dt = 0; dt < HD / 16; dt++) {
            uint32_t d = 16 * dt + 4 * g;
            if (d < hd)
                *(float4*)(o + d) = float4{R[t].o[dt][0] / R[t].l, R[t].o[dt][1] / R[t].l, R[t].o[dt][2] / R[t].l,
                                           R[t].o[dt][3] / R[t].l};
        }
    }
}

// ---------------------------------------------------------------------------------------
// The left fold of split chunks, in chunk order, then O / L. One workgroup per group:
// direct launches: (item, KV head); shared launches: (KV head, row block).
template <int HD>
__global__ __launch_bounds__(256) void attn_combine(const CombineParams p) {
    const uint32_t grp = blockIdx.x;
    const uint32_t hd = p.hd;
    uint32_t unit0, nchunk, nslot, kvh;
    uint32_t item = 0, rbi = 0;
    if (p.shared) {
        kvh = grp / p.nrb;
        rbi = grp % p.nrb;
        unit0 = grp * p.nchunk;
        nchunk = p.nchunk;
        nslot = p.slots;
    } else {
        item = grp / p.nkv;
        kvh = grp % p.nkv;
        unit0 = p.items[item].unit0 + kvh * p.items[item].nchunk;
        nchunk = p.items[item].nchunk;
        nslot = p.G;
    }
    for (uint32_t e = threadIdx.x; e < nslot * hd; e += blockDim.x) {
        uint32_t sl = e / hd, d = e % hd;
        uint32_t r, h;
        if (p.shared) {
            uint32_t gh = sl / p.rb, rl = sl % p.rb;
            r = rbi * p.rb + rl;
            if (gh >= p.G || rl >= p.rb || r >= p.rows) continue;
            h = kvh * p.G + gh;
        } else {
            r = p.items[item].row;
            h = kvh * p.G + sl;
        }
        float M = -INFINITY, L = 0.0f, O = 0.0f;
        for (uint32_t c = 0; c < nchunk; c++) {
            size_t at = (size_t)(unit0 + c) * p.slots + sl;
            float2 ml = *(const float2*)(p.part_ml + at * 2);
            float o = p.part_o[at * HD + d];
            float a, b, mn;
            merge_coef(M, ml.x, a, b, mn);
            L = L * a + ml.y * b;
            O = O * a + o * b;
            M = mn;
        }
        p.out[((size_t)r * p.nh + h) * hd + d] = O / L;
    }
}

// ---------------------------------------------------------------------------------------
// Launch plans.

static uint32_t ceil_div(uint64_t a, uint64_t b) { return (uint32_t)((a + b - 1) / b); }

// Chunk of a one-row call: about 128 chunks of the list, 64..256 entries, so a decode step
// fills the CUs from a few thousand visible slots up; from 16385 on it is CHUNK_MULTI.
uint32_t decode_chunk(uint64_t len) {
    uint64_t want = (len + 127) / 128;
    uint32_t c = 64;
    while (c < want && c < CHUNK_MULTI) c <<= 1;
    return c;
}

template <int HD, typename KVT>
static hipError_t launch_direct_t(DirectParams& dp, uint32_t units, hipStream_t s) {
    hipLaunchKernelGGL((attn_direct<HD, KVT>), dim3(units), dim3(64), 0, s, dp);
    return hipGetLastError();
}

template <int HD>
static hipError_t launch_combine_t(const CombineParams& cp, uint32_t groups, hipStream_t s) {
    hipLaunchKernelGGL((attn_combine<HD>), dim3(groups), dim3(256), 0, s, cp);
    return hipGetLastError();
}

template <int HD, typename KVT, int W, int NT>
static hipError_t launch_shared_t(const SharedParams& sp, uint32_t blocks, hipStream_t s) {
    hipLaunchKernelGGL((attn_shared<HD, KVT, W, NT>), dim3(blocks), dim3(64 * W), 0, s, sp);
    return hipGetLastError();
}

static int pad_hd(uint32_t hd) {
    if (hd <= 32) return 32;
    if (hd <= 64) return 64;
    if (hd <= 128) return 128;
    return 256;
}

#define BCHIP_DISPATCH_HD(hdp, CALL)            \
    switch (hdp) {                              \
        case 32: { constexpr int HD = 32; CALL; } break;   \
        case 64: { constexpr int HD = 64; CALL; } break;   \
        case 128: { constexpr int HD = 128; CALL; } break; \
        default: { constexpr int HD = 256; CALL; } break;  \
    }

hipError_t direct_attention(const AttnCall& a, const Item* items, uint32_t nitems,
                            Workspace& ws, hipStream_t s) {
    DirectParams dp{};
    dp.q = a.q;
    dp.kc = a.kc;
    dp.vc = a.vc;
    dp.out = a.out;
    dp.nh = a.nh;
    dp.nkv = a.nkv;
    dp.hd = a.hd;
    dp.G = a.nh / a.nkv;
    dp.masks = a.masks;
    dp.slot_limit = a.slot_limit;
    dp.base = a.pos;
    dp.tree = a.tree;
    dp.sc = a.scale * LOG2E;
    dp.nitems = nitems;
    uint64_t total_chunks = 0;
    for (uint32_t i = 0; i < nitems; i++) total_chunks += items[i].nchunk;
    // Split by chunk unless the launch already has plenty of waves.
    dp.split = (total_chunks > nitems) && (uint64_t)nitems * a.nkv < 1024;
    uint32_t units = 0;
    for (uint32_t i = 0; i < nitems; i++) {
        dp.items[i] = items[i];
        dp.items[i].unit0 = units;
        units += a.nkv * (dp.split ? items[i].nchunk : 1u);
    }
    const int hdp = pad_hd(a.hd);
    if (dp.split) {
        hipError_t e = ws.reserve((size_t)units * 16, (size_t)hdp);
        if (e != hipSuccess) return e;
        dp.part_o = ws.o;
        dp.part_ml = ws.ml;
    }
    hipError_t e;
    if (a.kv_type == 1) {
        BCHIP_DISPATCH_HD(hdp, e = (launch_direct_t<HD, f16>(dp, units, s)));
    } else {
        BCHIP_DISPATCH_HD(hdp, e = (launch_direct_t<HD, float>(dp, units, s)));
    }
    if (e != hipSuccess || !dp.split) return e;
    CombineParams cp{};
    cp.out = a.out;
    cp.part_o = ws.o;
    cp.part_ml = ws.ml;
    cp.nh = a.nh;
    cp.nkv = a.nkv;
    cp.hd = a.hd;
    cp.G = dp.G;
    cp.slots = 16;
    cp.shared = 0;
    cp.nitems = nitems;
    for (uint32_t i = 0; i < nitems; i++) cp.items[i] = dp.items[i];
    BCHIP_DISPATCH_HD(hdp, e = (launch_combine_t<HD>(cp, nitems * a.nkv, s)));
    return e;
}

hipError_t shared_attention(const AttnCall& a, Workspace& ws, hipStream_t s) {
    SharedParams sp{};
    sp.q = a.q;
    sp.kc = a.kc;
    sp.vc = a.vc;
    sp.out = a.out;
    sp.rows = a.rows;
    sp.nh = a.nh;
    sp.nkv = a.nkv;
    sp.hd = a.hd;
    sp.G = a.nh / a.nkv;
    sp.pos = a.pos;
    sp.sc = a.scale * LOG2E;
    const int hdp = pad_hd(a.hd);
    // Small batches (verify): 64 slots a workgroup; large (prefill): 128.
    const bool wide = (uint64_t)a.rows * sp.G > 64 && hdp <= 128;
    const uint32_t SL = wide ? 128u : 64u;
    sp.rb = SL / sp.G;
    if (sp.rb > a.rows) sp.rb = a.rows;
    sp.nrb = ceil_div(a.rows, sp.rb);
    const uint64_t maxlen = (uint64_t)a.pos + a.rows;
    sp.nchunk = ceil_div(maxlen, CHUNK_MULTI);
    const uint32_t groups = a.nkv * sp.nrb;
    sp.split = groups < 512 && sp.nchunk > 1;
    if (sp.split) {
        hipError_t e = ws.reserve((size_t)groups * sp.nchunk * SL, (size_t)hdp);
        if (e != hipSuccess) return e;
        sp.part_o = ws.o;
        sp.part_ml = ws.ml;
    }
    const uint32_t blocks = groups * (sp.split ? sp.nchunk : 1u);
    hipError_t e;
    if (a.kv_type == 1) {
        if (wide) {
            BCHIP_DISPATCH_HD(hdp, e = (launch_shared_t<HD, f16, 4, (HD <= 128 ? 2 : 1)>(sp, blocks, s)));
        } else {
            BCHIP_DISPATCH_HD(hdp, e = (launch_shared_t<HD, f16, 4, 1>(sp, blocks, s)));
        }
    } else {
        if (wide) {
            BCHIP_DISPATCH_HD(hdp, e = (launch_shared_t<HD, float, 4, (HD <= 128 ? 2 : 1)>(sp, blocks, s)));
        } else {
            BCHIP_DISPATCH_HD(hdp, e = (launch_shared_t<HD, float, 4, 1>(sp, blocks, s)));
        }
    }
    if (e != hipSuccess || !sp.split) return e;
    CombineParams cp{};
    cp.out = a.out;
    cp.part_o = ws.o;
    cp.part_ml = ws.ml;
    cp.nh = a.nh;
    cp.nkv = a.nkv;
    cp.hd = a.hd;
    cp.G = sp.G;
    cp.slots = SL;
    cp.shared = 1;
    cp.rows = a.rows;
    cp.rb = sp.rb;
    cp.nrb = sp.nrb;
    cp.nchunk = sp.nchunk;
    BCHIP_DISPATCH_HD(hdp, e = (launch_combine_t<HD>(cp, groups, s)));
    return e;
}

}  // namespace bchip
