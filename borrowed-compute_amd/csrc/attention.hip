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
// the row's result is the left fold of its chunks' (m, l, O) (merge below). The same
// arithmetic computes every chunk, whichever workgroup runs it, so a chunk can run on any
// CU and the row's bits do not change:
//  - attn_decode: four waves split each block (wave w scores key tile w and owns hd slice
//    w of the values), exchanging maxima, sums and P through LDS; the next block's K and V
//    are in flight while one is computed. The G heads of one row per workgroup: one-row
//    decode (split across CUs by chunk), ragged multi-sequence decode, and tree rows (each
//    row gathers its own list).
//  - attn_shared: four waves share K/V blocks staged in LDS (double-buffered) for up to
//    128 slots (rows x G heads of one KV head): prefill and line verify.
//  - attn_combine: the left fold of split chunks, in chunk order; the fold weights depend
//    only on the running maxima, so they are computed for all chunks at once (a prefix
//    max), leaving a three-operation recurrence per output.
// Every product of the fold, the softmax and the normalisation rounds on its own (the
// library is built with -ffp-contract=off), so each step is the same bits in every kernel.
#include "common.hpp"
#include "internal.hpp"

#include <hip/hip_ext.h>
#include <math.h>
#include <algorithm>
#include <type_traits>
#include <stdlib.h>

namespace bchip {

// f16 per row of the transposed V tile in LDS: 64 keys + 4 pad (8-byte aligned rows).

// Softmax state of the lane's slot over NDT output tiles of 16 dims.
template <int NDT>
struct State {
    f32x4 o[NDT];  // O^T[16*dt + 4*(lane/16) + i][lane%16]
    float m, l;    // running max (log2 units) and sum
};

template <int NDT>
__device__ __forceinline__ void state_clear(State<NDT>& s) {
#pragma unroll
    for (int i = 0; i < NDT; i++) s.o[i] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    s.m = -INFINITY;
    s.l = 0.0f;
}


// The running max of a slot moves only when a block's max passes it by more than LAZY
// (log2 units): until then the block's P = 2^(x - m) may reach 2^LAZY (exact in f16's
// range) and O and l keep their scale, so most blocks skip the rescale of O. Every kernel
// applies the same rule per slot, so a row's bits do not depend on which kernel, wave or
// neighbours computed it. mn: the new max; ms: the subtrahend of the block's exponents (0
// for a slot that has seen nothing); corr: the factor on O and l (exactly 1 when the max
// stays, 0 for a slot's first visible block).
constexpr float LAZY = 8.0f;

__device__ __forceinline__ void lazy_max(float m, float mx, float& mn, float& ms, float& corr) {
    const bool up = mx > m + LAZY;
    mn = up ? mx : m;
    ms = (mn == -INFINITY) ? 0.0f : mn;
    corr = up ? exp2_hw(m - ms) : 1.0f;
}

// R <- fold(R, c). attn_combine applies the same per-element expression.
template <int NDT>
__device__ __forceinline__ void fold(State<NDT>& R, const State<NDT>& c) {
    float a, b, mn;
    merge_coef(R.m, c.m, a, b, mn);
    R.l = R.l * a + c.l * b;
#pragma unroll
    for (int i = 0; i < NDT; i++) R.o[i] = R.o[i] * a + c.o[i] * b;
    R.m = mn;
}

// The two lane-group crossings of a 16-key tile: permlane swaps hand each lane the pair
// (x[l], x[l^16]) (or l^32) from the lower and the upper lane, in that order on both lanes,
// so a max or a sum of the pair is the same bits on both. A slot's sum over a 64-entry block
// is, per lane, a chain of dot2 steps over its f16 P values (pairs of keys, the four tiles
// in order), then the pairs across l^16, then across l^32.
__device__ __forceinline__ float xmax16(float x) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float xmax32(float x) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float xsum16(float x) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float xsum32(float x) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float tile_sum(float s) { return xsum32(xsum16(s)); }

// acc + h[0] + h[1] as one dot2 step with (1, 1): exact f16 products, one f32 accumulate.
__device__ __forceinline__ float pair_sum(half2 h, float acc) {
    return __builtin_amdgcn_fdot2(h, half2{(f16)1.0f, (f16)1.0f}, acc, false);
}
__device__ __forceinline__ float tile_max(float m) { return xmax32(xmax16(m)); }

// O <- O * corr for a wave's slots, skipped when every slot's max held (corr == 1 exactly,
// and x * 1 == x): in a long list the running max rarely moves, and the rescale is VALU
// work on every output register.
// keep_branch() marks a uniform branch's body as having an effect, so the compiler keeps
// the branch instead of running the body for every wave and selecting (which it otherwise
// does for short bodies, turning a skipped multiply into an executed one).
__device__ __forceinline__ void keep_branch() { asm volatile(""); }

template <int NDT>
__device__ __forceinline__ void rescale(f32x4 (&o)[NDT], float corr) {
    if (__all(corr == 1.0f)) return;
    keep_branch();
#pragma unroll
    for (int dt = 0; dt < NDT; dt++) o[dt] = o[dt] * corr;
}

// The V^T operand of one PV MFMA: lane (g, n) holds V[key(g, j)][16*dt + n] for the
// k-dimension order key(g, j) = 32*kc + 16*(j/4) + 4*g + j%4, the order in which this
// lane holds P^T after the score MFMAs.
// V tiles sit in LDS row-major ([key][dims], stride VS halves) and reach the MFMA A
// operand of O^T = V^T P^T through gfx950's transposing LDS read: within each 16-lane
// group, source lane j names row kbase + j/4, dims c0 + 4(j%4) .. +3, and result lane i
// receives dims c0 + i of rows kbase .. kbase+3. Lane (n, g) thus holds V[key][16dt + n] for
// keys 32kc + 4g + 0..3 (first half) and 32kc + 16 + 4g + 0..3 (second half): the key order
// of the P^T operand built from S^T's registers.
__device__ __forceinline__ half4 lds_tr4(const f16* p) {
    typedef short s16x4 __attribute__((ext_vector_type(4)));
    const s16x4 v = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) s16x4*)p);
    return __builtin_bit_cast(half4, v);
}

// Eight transposing reads (rows a_j and a_j + 16 rows of 256 bytes) and the wait for them,
// as one statement: the results exist only once it is done, so nothing can read them early,
// and the compiler adds no wait of its own (it would wait for every direct-to-LDS load in
// flight, not knowing these reads miss the stages still filling). The caller must know
// the rows' data has landed in LDS.
__device__ __forceinline__ void lds_tr4x4(half4 (&lo)[4], half4 (&hi)[4], uint32_t a0, uint32_t a1, uint32_t a2,
                                          uint32_t a3) {
    typedef short s16x4 __attribute__((ext_vector_type(4)));
    s16x4 l0, l1, l2, l3, h0, h1, h2, h3;
    asm volatile(
        "ds_read_b64_tr_b16 %0, %8\n\tds_read_b64_tr_b16 %4, %8 offset:4096\n\t"
        "ds_read_b64_tr_b16 %1, %9\n\tds_read_b64_tr_b16 %5, %9 offset:4096\n\t"
        "ds_read_b64_tr_b16 %2, %10\n\tds_read_b64_tr_b16 %6, %10 offset:4096\n\t"
        "ds_read_b64_tr_b16 %3, %11\n\tds_read_b64_tr_b16 %7, %11 offset:4096\n\t"
        "s_waitcnt lgkmcnt(0)"
        : "=&v"(l0), "=&v"(l1), "=&v"(l2), "=&v"(l3), "=&v"(h0), "=&v"(h1), "=&v"(h2), "=&v"(h3)
        : "v"(a0), "v"(a1), "v"(a2), "v"(a3));
    lo[0] = __builtin_bit_cast(half4, l0);
    lo[1] = __builtin_bit_cast(half4, l1);
    lo[2] = __builtin_bit_cast(half4, l2);
    lo[3] = __builtin_bit_cast(half4, l3);
    hi[0] = __builtin_bit_cast(half4, h0);
    hi[1] = __builtin_bit_cast(half4, h1);
    hi[2] = __builtin_bit_cast(half4, h2);
    hi[3] = __builtin_bit_cast(half4, h3);
}

template <int VS>
__device__ __forceinline__ half8 v_operand(const f16* __restrict__ vl, int dt, int kc, int g, int j) {
    const f16* src = vl + (32 * kc + 4 * g + (j >> 2)) * VS + 16 * dt + 4 * (j & 3);
    const half4 a = lds_tr4(src), b = lds_tr4(src + 16 * VS);
    return half8{a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]};
}

// Row stride (halves) of a V tile of dw dims in LDS: a multiple of 16 halves with an odd
// count of 32-byte units, so that the four rows one transposing read takes per 16 lanes,
// and the eight rows of each 32-lane half, fall on distinct banks.
constexpr int v_stride(int dw) { return ((dw / 16) & 1) ? dw : dw + 16; }

// One block of 64 list entries [key0, key0+64) for NT tiles of one wave.
// kop(kt, c) gives the K operand of key tile kt (keys key0+16kt..) and hd chunk c:
// lane (g, n) holds K[key0 + 16kt + n][32c + 8g .. +8]; vop(dt, kc) gives the V^T operand
// of output tile dt and key half kc (the order of v_operand).
// len[t] is the list length of this lane's slot in tile t (entries >= len are masked).
template <int HD, int NT, typename KOp, typename VOp>
__device__ __forceinline__ void block_step(State<HD / 16> (&s)[NT], const half8 (&qb)[NT][HD / 32], KOp kop,
                                           VOp vop, uint32_t key0, const uint32_t (&len)[NT]) {
    const int lane = threadIdx.x & 63;
    const int g = lane >> 4;
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
        // Scores are in log2 units already (the scale rides in Q). Entries at or past a
        // slot's list length are masked; a block every slot sees whole skips the test.
        float x[4][4];
        float mx = -INFINITY;
#pragma unroll
        for (int kt = 0; kt < 4; kt++)
#pragma unroll
            for (int i = 0; i < 4; i++) x[kt][i] = st[t][kt][i];
        if (!__all(key0 + BLK <= len[t])) {
            keep_branch();
#pragma unroll
            for (int kt = 0; kt < 4; kt++)
#pragma unroll
                for (int i = 0; i < 4; i++)
                    if (key0 + 16 * kt + 4 * g + i >= len[t]) x[kt][i] = -INFINITY;
        }
        // The block max: the lane's sixteen entries, then across lanes (a max is exact in
        // any order).
#pragma unroll
        for (int kt = 0; kt < 4; kt++)
#pragma unroll
            for (int i = 0; i < 4; i++) mx = fmaxf(mx, x[kt][i]);
        mx = tile_max(mx);
        float mn, ms, corr;
        lazy_max(s[t].m, mx, mn, ms, corr);
        // P in f16, and the block sum of those f16 values: per lane a chain of dot2 steps
        // over the pairs (keys 4g+0,1 and 4g+2,3 of each tile, tiles in order), then across
        // lanes (l^16, then l^32).
        float ls = 0.0f;
#pragma unroll
        for (int kt = 0; kt < 4; kt++) {
#pragma unroll
            for (int j = 0; j < 2; j++) {
                const half2 hp = half2{(f16)exp2_hw(x[kt][2 * j] - ms), (f16)exp2_hw(x[kt][2 * j + 1] - ms)};
                ls = pair_sum(hp, ls);
                pb[t][kt >> 1][(kt & 1) * 4 + 2 * j] = hp[0];
                pb[t][kt >> 1][(kt & 1) * 4 + 2 * j + 1] = hp[1];
            }
        }
        const float ps = tile_sum(ls);
        s[t].l = s[t].l * corr + ps;
        s[t].m = mn;
        rescale(s[t].o, corr);
    }
#pragma unroll
    for (int dt = 0; dt < HD / 16; dt++)
#pragma unroll
        for (int kc = 0; kc < 2; kc++) {
            half8 a = vop(dt, kc);
#pragma unroll
            for (int t = 0; t < NT; t++) s[t].o[dt] = mfma16(a, pb[t][kc], s[t].o[dt]);
        }
}

// 8 consecutive elements of a cache row, loaded now and converted to f16 where they are
// used (f32 caches round to nearest even), so that a load's wait falls at its use. Lanes
// with nothing to read load from a zero page instead of branching around the load: a
// branch would make the compiler wait for every load in flight, prefetches included.
template <typename KVT>
struct Raw;
template <>
struct Raw<f16> {
    half8 v;
    __device__ __forceinline__ void load(const f16* p) { v = *(const half8*)p; }
    // A load marked as streaming (read once: kept out of the caches' reuse).
    __device__ __forceinline__ void load_stream(const f16* p) { v = __builtin_nontemporal_load((const half8*)p); }
    // Eight f32 values as the cache would hold them.
    __device__ __forceinline__ void set(float4 x, float4 y) {
        v = half8{(f16)x.x, (f16)x.y, (f16)x.z, (f16)x.w, (f16)y.x, (f16)y.y, (f16)y.z, (f16)y.w};
    }
    __device__ __forceinline__ half8 get() const { return v; }
};
template <>
struct Raw<float> {
    float4 a, b;
    __device__ __forceinline__ void load(const float* p) {
        a = *(const float4*)p;
        b = *(const float4*)(p + 4);
    }
    __device__ __forceinline__ void load_stream(const float* p) {
        const f32x4 x = __builtin_nontemporal_load((const f32x4*)p), y = __builtin_nontemporal_load((const f32x4*)(p + 4));
        a = float4{x[0], x[1], x[2], x[3]};
        b = float4{y[0], y[1], y[2], y[3]};
    }
    __device__ __forceinline__ void set(float4 x, float4 y) {
        a = x;
        b = y;
    }
    __device__ __forceinline__ half8 get() const {
        return half8{(f16)a.x, (f16)a.y, (f16)a.z, (f16)a.w, (f16)b.x, (f16)b.y, (f16)b.z, (f16)b.w};
    }
};

// 8 elements of a Q row times sc (the attention scale times log2(e), so that scores come
// out of the MFMA in exp2 units), rounded to f16: the B operand of the score MFMAs.
// The product is rounded to f32 and then to f16 in every kernel: the empty asm keeps the
// compiler from folding multiply and conversion into one mixed-precision FMA
// (v_fma_mixlo_f16), which rounds the exact product to f16 once and so differs from the
// two roundings in rare elements (it did so in some kernels and not others, by register
// allocation, which broke bit-identity between kernels that share this arithmetic).
__device__ __forceinline__ f16 scaled_f16(float x, float sc) {
    float y = x * sc;
    asm("" : "+v"(y));
    return (f16)y;
}
__device__ __forceinline__ half8 q_scaled(float4 a, float4 b, float sc) {
    return half8{scaled_f16(a.x, sc), scaled_f16(a.y, sc), scaled_f16(a.z, sc), scaled_f16(a.w, sc),
                 scaled_f16(b.x, sc), scaled_f16(b.y, sc), scaled_f16(b.z, sc), scaled_f16(b.w, sc)};
}

__device__ __forceinline__ half8 q_operand(const float* __restrict__ qrow, uint32_t hd0, uint32_t hd, bool ok, float sc) {
    if (!ok || hd0 >= hd) return half8{0, 0, 0, 0, 0, 0, 0, 0};
    float4 a = *(const float4*)(qrow + hd0), b = *(const float4*)(qrow + hd0 + 4);
    return q_scaled(a, b, sc);
}

// Writes the 8 f16 values of key kl, dims d0..d0+7, into the row-major V tile vl.
template <int VS>
__device__ __forceinline__ void v_store(f16* __restrict__ vl, int kl, uint32_t d0, half8 v) {
    *(half8*)&vl[kl * VS + d0] = v;
}

// ---------------------------------------------------------------------------------------
// Decode kernel: the G query heads of one row against one KV head for one chunk of the
// row's list, four waves splitting every block. It writes the chunk's softmax state
// (m, l, O), or, for a row of one chunk, the normalised output; attn_combine folds the
// chunk states of multi-row passes (tree rows, a few line rows) left to right.
template <int NDT>
__device__ __forceinline__ void store_state(const State<NDT>& st, float* o_row, float* ml, uint32_t d0, uint32_t hd,
                                            int g, bool write_ml) {
#pragma unroll
    for (int dt = 0; dt < NDT; dt++) {
        const uint32_t d = d0 + 16 * dt + 4 * g;
        if (d < hd) *(float4*)(o_row + d) = float4{st.o[dt][0], st.o[dt][1], st.o[dt][2], st.o[dt][3]};
    }
    if (write_ml) *(float2*)ml = float2{st.m, st.l};
}

template <int HD, typename KVT>
__global__ __launch_bounds__(256, sizeof(KVT) == 2 && HD <= 128 ? 4 : 2) void attn_decode(const DirectParams p) {
    constexpr int NDT = HD / 16;                     // output tiles of 16 dims
    constexpr int DTW = NDT >= 4 ? NDT / 4 : 1;      // output tiles per wave
    constexpr int DW = 16 * DTW;                     // dims per wave
    constexpr int LPK = DW / 8;                      // lanes per key in a V load (8 elements each)
    constexpr int KPI = 64 / LPK;                    // keys per V load
    constexpr int NVL = BLK / KPI;                   // V loads per block
    constexpr int NKC = HD / 32;                     // K loads per block (hd chunks)
    constexpr int VSW = v_stride(DW);
    __shared__ __attribute__((aligned(16))) f16 vt[4][BLK * VSW];
    __shared__ float red[2][4][16];                  // [parity][key tile][slot]: tile maxes
    __shared__ __attribute__((aligned(8))) half4 pt[2][4][4][16];  // [parity][key tile][g][slot]
    __shared__ __attribute__((aligned(16))) half8 qs[NKC][64];     // Q^T operands by lane
    __shared__ uint32_t tail[64];
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int g = lane >> 4, n = lane & 15;
    const bool pv = w * DTW < NDT;  // waves with an hd slice (all but for hd <= 32)
    const uint32_t d0 = 16 * DTW * w;
    const uint32_t hd = p.hd, kvd = p.nkv * hd;
    const KVT* zp = (const KVT*)p.zero;

    // One unit per workgroup (tree rows), in (item, chunk, KV head) order: the KV heads of
    // one chunk read one stretch of the cache together. Consecutive workgroups go to the 8 XCDs in
    // turn, so the KV head turns with the chunk (j + c) to give every XCD a mix of heads:
    // a fixed head per XCD leaves the XCDs whose head's cache columns map to busier HBM
    // channels finishing last. The state is stored at the unit's canonical index.
    const uint32_t u = blockIdx.x;
    uint32_t it = 0;
    if (p.nitems > 1) {
        // The last item whose first unit is at or below u (items hold their units in order),
        // every item's first unit read by one lane at once (MAX_ITEMS is the wave size).
        const uint32_t u0 = p.items[(uint32_t)lane < p.nitems ? lane : 0].unit0;
        it = (uint32_t)__popcll(__ballot((uint32_t)lane < p.nitems && u0 <= u)) - 1u;
    }
    const Item I = p.items[it];
    const uint32_t rem = u - I.unit0, c = rem / p.nkv, kvh = (rem % p.nkv + c) % p.nkv;
    const size_t cu = (size_t)I.unit0 + (size_t)c * p.nkv + kvh;
    // Slot n of an item is row I.row + n / G, head kvh * G + n % G (an item is one tree
    // row: nrows = 1).
    const uint32_t srow = n / p.G, shead = kvh * p.G + n % p.G;
    const bool valid = srow < I.nrows;
    const KVT* kc = (const KVT*)p.kc + I.kvoff * kvd + (size_t)kvh * hd;
    const KVT* vc = (const KVT*)p.vc + I.kvoff * kvd + (size_t)kvh * hd;
    // The row's list: the slots below base, then base + j for each set bit j of its mask.
    const uint32_t lo = p.masks[2 * I.row], hi = p.masks[2 * I.row + 1];
    const uint32_t ntail = __popc(lo) + __popc(hi);
    const uint32_t len = p.base + ntail;
    if ((uint32_t)tid < ntail) tail[tid] = p.base + nth_set_bit(lo, hi, tid);
    __syncthreads();
    const uint32_t lane_len = len;  // this slot's list
    const uint32_t kb0 = c * I.chunk, kb1 = min(kb0 + I.chunk, len);

    // Cache slot of list entry k, or ok = false for entries past the list (and for tree
    // slots past the cache, which a bad mask could name): those read as zeros.
    auto slot_of = [&](uint32_t k, bool& ok) -> uint32_t {
        ok = k < len;
        if (!ok) return 0u;
        const uint32_t s = k < p.base ? k : tail[k - p.base];
        ok = (uint64_t)s + I.kvoff < p.slot_limit;
        return ok ? s : 0u;
    };
    // K and V of block key0 into registers; entries at or past kb1 read the zero page, so
    // the prefetch past the last block costs no HBM traffic and needs no branch.
    auto load_block = [&](uint32_t key0, Raw<KVT> (&kr)[NKC], Raw<KVT> (&vr)[NVL]) {
        bool ok;
        const uint32_t kk = key0 + 16 * w + n;
        const KVT* row = kc + (size_t)slot_of(kk, ok) * kvd;
        ok = ok && kk < kb1;
#pragma unroll
        for (int c2 = 0; c2 < NKC; c2++) {
            const uint32_t hd0 = 32 * c2 + 8 * g;
            kr[c2].load((ok && hd0 < hd) ? row + hd0 : zp);
        }
        const uint32_t d = d0 + 8 * (lane % LPK);
#pragma unroll
        for (int i = 0; i < NVL; i++) {
            const uint32_t kv = key0 + i * KPI + lane / LPK;
            const KVT* vrow = vc + (size_t)slot_of(kv, ok) * kvd;
            vr[i].load((pv && ok && kv < kb1 && d < hd) ? vrow + d : zp);
        }
    };
    // Two register sets in turn: the next block loads into one while the other is used, and
    // no value is copied between them (a copy would wait for the load).
    Raw<KVT> kA[NKC], vA[NVL], kB[NKC], vB[NVL];
    // Q^T operands: wave w loads hd chunks w, w+4, ..., issued ahead of the first block so
    // that they do not queue behind it; lanes past G or hd read the zero page.
    constexpr int QPW = (NKC + 3) / 4;
    float4 qa[QPW], qb[QPW];
    {
        const float* qrow = p.q + ((size_t)(I.row + (valid ? srow : 0u)) * p.nh + (valid ? shead : 0u)) * hd;
#pragma unroll
        for (int j = 0; j < QPW; j++) {
            const uint32_t c2 = w + 4 * j, hd0 = 32 * c2 + 8 * g;
            const float* src = (c2 < (uint32_t)NKC && valid && hd0 < hd) ? qrow + hd0 : (const float*)p.zero;
            qa[j] = *(const float4*)src;
            qb[j] = *(const float4*)(src + 4);
        }
    }
    load_block(kb0, kA, vA);
#pragma unroll
    for (int j = 0; j < QPW; j++) {
        const uint32_t c2 = w + 4 * j;
        if (c2 < (uint32_t)NKC)
            qs[c2][lane] = q_scaled(qa[j], qb[j], p.sc);
    }
    __syncthreads();

    State<DTW> cs;
    state_clear(cs);
    int par = 0;
    auto compute_block = [&](uint32_t key0, const Raw<KVT> (&kr)[NKC], const Raw<KVT> (&vr)[NVL]) {
        // Scores of key tile w.
        f32x4 st = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int c2 = 0; c2 < NKC; c2++) st = mfma16(kr[c2].get(), qs[c2][lane], st);
        float x[4], tm = -INFINITY;
#pragma unroll
        for (int i = 0; i < 4; i++) x[i] = st[i];
        if (!__all(key0 + BLK <= lane_len)) {
            keep_branch();
#pragma unroll
            for (int i = 0; i < 4; i++)
                if (key0 + 16 * w + 4 * g + i >= lane_len) x[i] = -INFINITY;
        }
#pragma unroll
        for (int i = 0; i < 4; i++) tm = fmaxf(tm, x[i]);
        tm = tile_max(tm);
        if (g == 0) red[par][w][n] = tm;
        if (pv) {
#pragma unroll
            for (int i = 0; i < NVL; i++) v_store<VSW>(vt[w], i * KPI + lane / LPK, 8 * (lane % LPK), vr[i].get());
        }
        __syncthreads();
        const float mx = fmaxf(fmaxf(red[par][0][n], red[par][1][n]), fmaxf(red[par][2][n], red[par][3][n]));
        float mn, ms, corr;
        lazy_max(cs.m, mx, mn, ms, corr);
        half4 ph;
#pragma unroll
        for (int i = 0; i < 4; i++) ph[i] = (f16)exp2_hw(x[i] - ms);
        pt[par][w][g][n] = ph;
        __syncthreads();
        // The block sum in the multi-row order: per lane the dot2 chain over the four tiles'
        // pairs in order (every wave reads all four tiles of its lane), then across lanes.
        float ls = 0.0f;
#pragma unroll
        for (int t = 0; t < 4; t++) {
            const half4 h4 = pt[par][t][g][n];
            ls = pair_sum(half2{h4[0], h4[1]}, ls);
            ls = pair_sum(half2{h4[2], h4[3]}, ls);
        }
        const float ps = tile_sum(ls);
        cs.l = cs.l * corr + ps;
        cs.m = mn;
        if (pv) {
            rescale(cs.o, corr);
#pragma unroll
            for (int dt = 0; dt < DTW; dt++) {
                f32x4 o = cs.o[dt];
#pragma unroll
                for (int kc2 = 0; kc2 < 2; kc2++) {
                    const half4 a = pt[par][2 * kc2][g][n], b = pt[par][2 * kc2 + 1][g][n];
                    const half8 pb = half8{a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]};
                    o = mfma16(v_operand<VSW>(vt[w], dt, kc2, g, n), pb, o);
                }
                cs.o[dt] = o;
            }
        }
        par ^= 1;
    };
    if (kb0 < kb1) {
        for (uint32_t key0 = kb0;;) {
            load_block(key0 + BLK, kB, vB);
            compute_block(key0, kA, vA);
            key0 += BLK;
            if (key0 >= kb1) break;
            load_block(key0 + BLK, kA, vA);
            compute_block(key0, kB, vB);
            key0 += BLK;
            if (key0 >= kb1) break;
        }
    }
    if (!valid || !pv) return;
    if (I.nchunk == 1) {
        float* orow = p.out + ((size_t)(I.row + srow) * p.nh + shead) * hd;
#pragma unroll
        for (int dt = 0; dt < DTW; dt++) {
            const uint32_t d = d0 + 16 * dt + 4 * g;
            if (d < hd)
                *(float4*)(orow + d) =
                    float4{cs.o[dt][0] / cs.l, cs.o[dt][1] / cs.l, cs.o[dt][2] / cs.l, cs.o[dt][3] / cs.l};
        }
    } else {
        store_state(cs, p.part_o + (cu * 16 + n) * HD, p.part_ml + (cu * 16 + n) * 2, d0, hd, g,
                    w == 0 && g == 0);
    }
}

// ---------------------------------------------------------------------------------------
// One-row kernel (decode steps and ragged batches of them). A one-row list is bound only to
// be deterministic and within rounding of the same row in a batch, so it need not share the
// multi-row arithmetic: each wave streams one (chunk, KV head) unit alone, in blocks of RB
// entries, with no barrier and no exchange between waves. Lane (n, g) holds slot n (query
// head kvh * G + n) of keys 4g..4g+3 of each 16-key tile; the block's max and sum cross the
// four lane groups by permlane swaps, which hand every lane the pair (x[l], x[l^16]) or
// (x[l], x[l^32]) in the same order. K and V go through the wave's own LDS rows (loaded
// row-contiguous), K comes back in the score operands' layout and V transposed. The list's
// last entry (a fused step's new row) is a block of its own at the end of the last chunk.
// The four waves of a workgroup take consecutive units, four KV heads of one
// chunk, so a workgroup reads 4 * hd contiguous elements of every row it streams (measured
// faster than four chunks of one head: 25.5 against 30.9 us at 32768 slots x 8 KV heads).
// A unit whose chunk is the whole list writes the output; otherwise its state goes to the
// workspace and attn_row_fold combines a row's chunks. (Folding in the last workgroup to
// finish, found by an arrival counter, would save that launch, but publishing each state
// takes a device-scope release, an L2 write-back per workgroup: measured at +8 us for 256
// workgroups and +175 us for 4096 on MI355X.)
// The fold's order is fixed by the list alone: runs of ROW_RUN consecutive chunks, each
// folded left to right from a cleared state, then attn_row_fold's order over the runs. A
// launch of many units (RUNS: a ragged batch, whose lists keep the chunks they would have
// alone) gives each wave a whole run: it folds the run's chunks itself, in that order, and
// writes one state a run (an eighth of the states written and read back); the bits are
// those of a unit a chunk. Runs of eight against four: configs[3]'s ragged call 127.2 ->
// 125.3 us (medians of four interleaved runs), the 32768-slot step unchanged (28.5-28.7).
constexpr int RB = 32;                     // list entries per block of the one-row kernel
constexpr uint32_t ROW_FUSE_MAXG = 8;      // query heads per KV head a fused step takes
constexpr uint32_t ROW_MAX_CHUNKS = 256;   // chunks per (item, KV head): attn_row_fold's reach
constexpr uint32_t ROW_RUN = 8;            // chunks a run

template <int HD, typename KVT, bool FUSE, bool RUNS>
__global__ __launch_bounds__(256, 2) void attn_decode_row(const DirectParams p) {
    constexpr int NKC = HD / 32;        // hd chunks of a score MFMA
    constexpr int NDT = HD / 16;        // output tiles of 16 dims
    constexpr int VS = v_stride(HD);    // LDS row stride of V (halves)
    constexpr int VLR = HD / 8;         // lanes per V row (8 elements each)
    constexpr int VRI = 64 / VLR;       // V rows per load
    constexpr int NVL = RB / VRI;       // V loads per block
    __shared__ __attribute__((aligned(16))) f16 vl[4][RB * VS];
    // K through LDS where it fits beside V (f16, hd <= 128): K then loads as V does, 16 lanes
    // over a row's contiguous bytes, and the score operands come from the LDS tile (measured
    // faster than loading the operands straight into registers, 16 rows by 64 bytes a load:
    // 25.9 against 28.0 us at 32768 slots x 8 KV heads, and 131 against 154 us for the
    // ragged batch).
    constexpr bool KL = sizeof(KVT) == 2 && HD <= 128;
    constexpr int KS = HD + 8;  // LDS row stride of K (halves): rows 4 banks apart (pads of 4, 16, 24 measured slower)
    __shared__ __attribute__((aligned(16))) f16 kt[KL ? 4 : 1][KL ? RB * KS : 8];
    // The list's last entry (a fused step's new row) as the cache holds it, per wave: K then
    // V, dims past hd zero. The chunk that holds it takes it as a block of its own, after
    // its other entries, from here.
    __shared__ __attribute__((aligned(16))) KVT lrow[4][2][HD];
    // The wave index is uniform: every bound derived from it below (the unit, its chunk and
    // KV head, the block loop's end) stays in scalar registers, so the loop's exit is a
    // scalar branch and the loads of the next block need not wait for those in flight.
    const int tid = threadIdx.x, lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int g = lane >> 4, n = lane & 15;
    const uint32_t u = blockIdx.x * 4u + w;  // this wave's unit
    // The arguments are read before any branch on them, so that their scalar loads go out
    // together (one round trip to memory at the start rather than one for the unit count,
    // one for the item count and one for the item); a launch of one item needs no search.
    const uint32_t nunits = p.nunits, nitems = p.nitems;
    Item I = p.items[0];
    const uint32_t hd = p.hd, kvd = p.nkv * hd, G = p.G;
    asm volatile("" ::"s"(nunits), "s"(nitems), "s"(I.row), "s"(I.len), "s"(I.unit0), "s"(I.nchunk), "s"(I.chunk),
                 "s"(I.kvoff), "s"(hd), "s"(kvd), "s"(G), "s"(p.kc), "s"(p.vc), "s"(p.q), "s"(p.positions), "s"(p.zero),
                 "s"(p.nh), "s"(p.sc), "s"(p.knew), "s"(p.vnew), "s"(p.inv_freq), "s"(p.rope_dim), "s"(p.neox));
    if (u >= nunits) return;  // no barrier below: a wave may leave alone
    uint32_t it = 0;
    if (nitems > 1) {
        // The unit's item: the last whose first unit is at or below u (items hold their
        // units in order), every item's first unit read by one lane at once (MAX_ITEMS is
        // the wave size).
        const uint32_t u0 = p.items[(uint32_t)lane < nitems ? lane : 0].unit0;
        it = (uint32_t)__popcll(__ballot((uint32_t)lane < nitems && u0 <= u)) - 1u;
        I = p.items[it];
    }
    const uint32_t pos0 = FUSE ? p.positions[I.row] : 0u;  // before any store: a scalar load
    // The unit's chunks: one (uu), or with RUNS run uu's chunks cfirst .. cend - 1.
    const uint32_t rem = u - I.unit0, uu = rem / p.nkv, kvh = rem % p.nkv;
    const uint32_t cfirst = RUNS ? uu * ROW_RUN : uu;
    const uint32_t cend = RUNS ? min(cfirst + ROW_RUN, I.nchunk) : cfirst + 1;
    // The last chunk streams up to the list's last entry and then takes that entry alone:
    // the same blocks whether the entry came from the cache or, in a fused step, from this
    // kernel's own rotation (so both give the same bits), and no block of the stream holds a
    // slot this kernel writes.
    const uint32_t last = I.len - 1;
    const bool unit_last = min(cend * I.chunk, I.len) == I.len;  // the unit takes the list's last chunk
    // The chunk being streamed: its entries kb0 .. kb1 - 1, streamed up to kbs.
    uint32_t kb0, kb1, kbs;
    bool has_last;
    auto set_chunk = [&](uint32_t c) {
        kb0 = c * I.chunk;
        kb1 = min(kb0 + I.chunk, I.len);
        has_last = kb1 == I.len;
        kbs = has_last ? last : kb1;
    };
    set_chunk(cfirst);
    const bool valid = (uint32_t)n < G;
    const KVT* zp = (const KVT*)p.zero;
    const KVT* kc = (const KVT*)p.kc + I.kvoff * kvd + (size_t)kvh * hd;
    const KVT* vc = (const KVT*)p.vc + I.kvoff * kvd + (size_t)kvh * hd;

    // Block key0's K or V into registers; entries at or past kbs read the zero page (no HBM
    // traffic, no branch between the loads).
    auto load_k = [&](uint32_t key0, Raw<KVT> (&kr)[2][NKC]) {
        if constexpr (KL) {
            // Row-contiguous: load i holds entry key0 + i VRI + lane / VLR, dims 8 (lane % VLR).
            const uint32_t d = 8 * (lane % VLR);
#pragma unroll
            for (int i = 0; i < NVL; i++) {
                const uint32_t key = key0 + i * VRI + lane / VLR;
                kr[i / NKC][i % NKC].load_stream((key < kbs && d < hd) ? kc + (size_t)key * kvd + d : zp);
            }
            return;
        }
#pragma unroll
        for (int t = 0; t < 2; t++) {
            const uint32_t key = key0 + 16 * t + n;
            const KVT* row = kc + (size_t)(key < kbs ? key : 0u) * kvd;
#pragma unroll
            for (int c2 = 0; c2 < NKC; c2++) {
                const uint32_t hd0 = 32 * c2 + 8 * g;
                kr[t][c2].load_stream((key < kbs && hd0 < hd) ? row + hd0 : zp);
            }
        }
    };
    auto load_v = [&](uint32_t key0, Raw<KVT> (&vr)[NVL]) {
        const uint32_t d = 8 * (lane % VLR);
#pragma unroll
        for (int i = 0; i < NVL; i++) {
            const uint32_t key = key0 + i * VRI + lane / VLR;
            vr[i].load_stream((key < kbs && d < hd) ? vc + (size_t)key * kvd + d : zp);
        }
    };
    // Prologue. Every small load (q, the RoPE frequencies, the new or the last K/V row) goes
    // out before the first blocks' loads, unconditionally (lanes with nothing to read load
    // the zero page): a wave's loads complete in issue order, and a load behind a branch
    // makes the compiler wait for all loads in flight where the branch joins. The rotation
    // of a fused step then runs while the blocks are in flight.
    half8 qb[NKC];  // Q^T operands (B of the score MFMAs)
    f16* vw = vl[w];
    const bool has_new = FUSE && unit_last;  // this unit writes the new row
    constexpr bool DB = sizeof(KVT) == 2 && HD <= 128;
    constexpr int NLE = (HD + 63) / 64;                              // row elements per lane
    constexpr int NPJ = (HD / 2 + 63) / 64;                          // RoPE pairs per lane
    constexpr int NQL = FUSE ? ((int)ROW_FUSE_MAXG * HD + 255) / 256 : 1;  // q float4s per lane
    constexpr int MG = FUSE ? (int)ROW_FUSE_MAXG : 1;
    const uint32_t half = hd / 2;
    const float* zf = (const float*)p.zero;
    KVT lk[NLE], lv[NLE];     // !FUSE: the last entry, from the cache
    float4 qa[NKC], qc[NKC];  // !FUSE: q
    float fr[NPJ];            // FUSE: frequencies of this lane's pairs
    // FUSE: the G heads' q (qs [G][hd] in the wave's LDS tile), the new k (ks) and v (vs),
    // 16 bytes a lane per load; the rotation works in LDS.
    float* qs = (float*)vw;
    float* ks = qs + NQL * 256;
    float* vs = ks + 256;
    static_assert(!FUSE || (NQL * 256 + 512) * 4 <= RB * VS * 2, "the fused prologue's q, k, v fit the wave's tile");
    f32x4 qf[NQL], kf, vf;
    if constexpr (FUSE) {
#pragma unroll
        for (int j = 0; j < NPJ; j++) {
            const uint32_t pp = lane + 64 * j;
            fr[j] = *(pp < p.rope_dim / 2 ? p.inv_freq + pp : zf);
        }
        const float* qg = p.q + ((size_t)I.row * p.nh + kvh * G) * hd;
#pragma unroll
        for (int i = 0; i < NQL; i++) {
            const uint32_t e = 4 * (lane + 64 * i);
            qf[i] = *(const f32x4*)(e < G * hd ? qg + e : zf);
        }
        const bool nk = has_new && 4 * (uint32_t)lane < hd;
        const size_t kvrow = ((size_t)I.row * p.nkv + kvh) * hd + 4 * lane;
        kf = *(const f32x4*)(nk ? p.knew + kvrow : zf);
        vf = *(const f32x4*)(nk ? p.vnew + kvrow : zf);
    } else {
#pragma unroll
        for (int j = 0; j < NLE; j++) {
            const uint32_t e = lane + 64 * j;
            const bool ok = unit_last && e < hd;
            lk[j] = *(ok ? kc + (size_t)last * kvd + e : zp);
            lv[j] = *(ok ? vc + (size_t)last * kvd + e : zp);
        }
        const float* qrow = p.q + ((size_t)I.row * p.nh + kvh * G + (valid ? n : 0)) * hd;
#pragma unroll
        for (int c2 = 0; c2 < NKC; c2++) {
            const uint32_t hd0 = 32 * c2 + 8 * g;
            const float* src = (valid && hd0 < hd) ? qrow + hd0 : zf;
            qa[c2] = *(const float4*)src;
            qc[c2] = *(const float4*)(src + 4);
        }
    }
    Raw<KVT> kR[2][2][NKC], vR[NVL], vR2[NVL];
    // A stream of at most two blocks (short lists) has all of it in flight through the
    // prologue; a longer one has the first block and the second block's K.
    bool two;
    auto first_loads = [&]() {
        two = kbs <= kb0 + 2 * RB;
        if constexpr (DB) {
            load_k(kb0, kR[0]);
            load_v(kb0, vR);
            load_k(kb0 + RB, kR[1]);
            if (two) load_v(kb0 + RB, vR2);
        }
    };
    first_loads();
    if constexpr (FUSE) {
        // q, k and v into the LDS tile; then each lane rotates its pairs there (the angle
        // depends on the pair alone, so its sine and cosine serve all G heads and the new K
        // row), and the operands come from there.
#pragma unroll
        for (int i = 0; i < NQL; i++) *(f32x4*)&qs[4 * (lane + 64 * i)] = qf[i];
        *(f32x4*)&ks[4 * lane] = kf;
        *(f32x4*)&vs[4 * lane] = vf;
        const float posf = (float)pos0;
        // All ROW_FUSE_MAXG heads' pairs at once (heads past G are the zeros their loads
        // read), so the LDS reads go out together; unrotated dims pass through unchanged.
#pragma unroll
        for (int j = 0; j < NPJ; j++) {
            const uint32_t pp = lane + 64 * j;
            const bool act = pp < half;
            uint32_t a, b;
            const bool rot = rope_pair(pp, p.rope_dim, p.neox, a, b) && act;
            if (!act) a = b = 0;
            float sn, cs;
            sincosf(posf * fr[j], &sn, &cs);  // fr = 0 where not rotated
            float x0[MG], x1[MG];
#pragma unroll
            for (int h = 0; h < MG; h++) {
                x0[h] = qs[h * hd + a];
                x1[h] = qs[h * hd + b];
            }
            if (act) {
#pragma unroll
                for (int h = 0; h < MG; h++) {
                    float y0, y1;
                    rotate_sc(x0[h], x1[h], sn, cs, y0, y1);
                    qs[h * hd + a] = rot ? y0 : x0[h];
                    qs[h * hd + b] = rot ? y1 : x1[h];
                }
            }
            if (has_new && act) {
                float y0 = ks[a], y1 = ks[b];
                if (rot) rotate_sc(ks[a], ks[b], sn, cs, y0, y1);
                const KVT k0 = to_kv<KVT>(y0), k1 = to_kv<KVT>(y1);
                KVT* kdst = (KVT*)p.kc + (I.kvoff + last) * kvd + (size_t)kvh * hd;
                kdst[a] = k0;
                kdst[b] = k1;
                lrow[w][0][a] = k0;
                lrow[w][0][b] = k1;
            }
        }
        if (has_new) {
            // V as the cache holds it, and zeros past hd in both rows.
            const uint32_t e = 4 * lane;
            if (e < (uint32_t)HD) {
                const KVT v0 = to_kv<KVT>(vs[e]), v1 = to_kv<KVT>(vs[e + 1]), v2 = to_kv<KVT>(vs[e + 2]),
                          v3 = to_kv<KVT>(vs[e + 3]);
                if (e < hd) {
                    KVT* vdst = (KVT*)p.vc + (I.kvoff + last) * kvd + (size_t)kvh * hd + e;
                    vdst[0] = v0;
                    vdst[1] = v1;
                    vdst[2] = v2;
                    vdst[3] = v3;
                } else {
                    lrow[w][0][e] = lrow[w][0][e + 1] = lrow[w][0][e + 2] = lrow[w][0][e + 3] = to_kv<KVT>(0.0f);
                }
                lrow[w][1][e] = v0;
                lrow[w][1][e + 1] = v1;
                lrow[w][1][e + 2] = v2;
                lrow[w][1][e + 3] = v3;
            }
        }
        // The operands: 16-byte LDS reads (hd is a multiple of 32 here), unconditional
        // (other lanes read head 0 and take zeros).
#pragma unroll
        for (int c2 = 0; c2 < NKC; c2++) {
            const uint32_t hd0 = 32 * c2 + 8 * g;
            const bool ok = valid && hd0 < hd;
            const float* src = (const float*)__builtin_assume_aligned(&qs[(valid ? n : 0) * hd + (hd0 < hd ? hd0 : 0)], 16);
            const f32x4 lo = *(const f32x4*)src, hi = *(const f32x4*)(src + 4);
            const half8 h = q_scaled(float4{lo[0], lo[1], lo[2], lo[3]}, float4{hi[0], hi[1], hi[2], hi[3]}, p.sc);
            qb[c2] = ok ? h : half8{0, 0, 0, 0, 0, 0, 0, 0};
        }
        // q stays rotated, as k_rope leaves it. Other units of this KV head may still be
        // reading it, so with several chunks the first one stages the rotated heads (at the
        // item's place in qrot) and attn_row_fold, which runs after every unit, copies them
        // into q; a lone unit writes q.
        if (cfirst == 0) {
            float* dst = (I.nchunk == 1 ? p.qw + (size_t)I.row * p.nh * hd : p.qrot + (size_t)it * p.nh * hd) +
                         (size_t)kvh * G * hd;
            for (uint32_t e = 4 * lane; e < G * hd; e += 256)
                *(f32x4*)&dst[e] = *(const f32x4*)__builtin_assume_aligned(&qs[e], 16);
        }
    } else {
#pragma unroll
        for (int c2 = 0; c2 < NKC; c2++) qb[c2] = q_scaled(qa[c2], qc[c2], p.sc);
        if (unit_last) {
#pragma unroll
            for (int j = 0; j < NLE; j++) {
                const uint32_t e = lane + 64 * j;
                if (e < (uint32_t)HD) {
                    lrow[w][0][e] = lk[j];
                    lrow[w][1][e] = lv[j];
                }
            }
        }
    }
    f32x4 o[NDT];
#pragma unroll
    for (int dt = 0; dt < NDT; dt++) o[dt] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    float m = -INFINITY, l = 0.0f;
    // One block of RB entries from key0; entries at or past `end` are masked. after_v runs
    // once the block's V is in LDS (its registers free), before the PV products.
    auto compute_block = [&](uint32_t key0, uint32_t end, const Raw<KVT> (&kr)[2][NKC], const Raw<KVT> (&vr)[NVL],
                             auto after_v) {
        f32x4 st[2];
        if constexpr (KL) {
            f16* kw = kt[KL ? w : 0];
#pragma unroll
            for (int i = 0; i < NVL; i++) *(half8*)&kw[(i * VRI + lane / VLR) * KS + 8 * (lane % VLR)] = kr[i / NKC][i % NKC].get();
#pragma unroll
            for (int t = 0; t < 2; t++) {
                st[t] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
                for (int c2 = 0; c2 < NKC; c2++)
                    st[t] = mfma16(*(const half8*)&kw[(16 * t + n) * KS + 32 * c2 + 8 * g], qb[c2], st[t]);
            }
        } else {
#pragma unroll
            for (int t = 0; t < 2; t++) {
                st[t] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
                for (int c2 = 0; c2 < NKC; c2++) st[t] = mfma16(kr[t][c2].get(), qb[c2], st[t]);
            }
        }
        float x[2][4], mx = -INFINITY;
#pragma unroll
        for (int t = 0; t < 2; t++)
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const uint32_t k = key0 + 16 * t + 4 * g + i;
                x[t][i] = (k < end) ? st[t][i] : -INFINITY;
                mx = fmaxf(mx, x[t][i]);
            }
        mx = xmax32(xmax16(mx));
        float mn, ms, corr;
        lazy_max(m, mx, mn, ms, corr);
        half8 pb;
        float ts = 0.0f;
#pragma unroll
        for (int t = 0; t < 2; t++)
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const f16 e = (f16)exp2_hw(x[t][i] - ms);
                ts = ts + (float)e;
                pb[4 * t + i] = e;
            }
        ts = xsum32(xsum16(ts));
        l = l * corr + ts;
        m = mn;
#pragma unroll
        for (int i = 0; i < NVL; i++) v_store<VS>(vw, i * VRI + lane / VLR, 8 * (lane % VLR), vr[i].get());
        after_v();
        rescale(o, corr);
#pragma unroll
        for (int dt = 0; dt < NDT; dt++) o[dt] = mfma16(v_operand<VS>(vw, dt, 0, g, n), pb, o[dt]);
    };
    auto nothing = [] {};
    // Where two K register sets fit (f16, hd <= 128), the loads run one block ahead in halves:
    // the next block's K goes out before this block's scores, its V once this block's V is in
    // LDS. About one block per wave is in flight at any time, beside the compute; a deeper
    // prefetch measured slower (more requests in flight than the memory system serves
    // best). Wider rows load and compute one block at a time; the other resident waves of
    // the CU still overlap them.
    // The streamed chunk's blocks, then (the list's last chunk) its last entry.
    auto stream = [&]() {
        if constexpr (DB) {
            // The first block, then two blocks per trip and one exit, at the bottom: with an exit
            // after every block the compiler merges the exits into one block that also leads back
            // to the loop's top, and must then assume loads of every register set are still in
            // flight there. A chunk with an even block count computes one block past its end: its
            // entries are all masked (P = 0 exactly, the max and the scale hold), its loads read
            // the zero page, and the state comes out unchanged.
            if (two) {
                compute_block(kb0, kbs, kR[0], vR, nothing);
                if (kb0 + RB < kbs) compute_block(kb0 + RB, kbs, kR[1], vR2, nothing);
            } else {
                compute_block(kb0, kbs, kR[0], vR, [&] { load_v(kb0 + RB, vR); });
            }
            for (uint32_t key0 = two ? kbs : kb0 + RB; key0 < kbs; key0 += 2 * RB) {
    #pragma unroll
                for (int s = 0; s < 2; s++) {
                    const uint32_t kb = key0 + s * RB;
                    load_k(kb + RB, kR[s]);
                    compute_block(kb, kbs, kR[1 - s], vR, [&] { load_v(kb + RB, vR); });
                }
            }
        } else {
            for (uint32_t key0 = kb0; key0 < kbs; key0 += RB) {
                load_k(key0, kR[0]);
                load_v(key0, vR);
                compute_block(key0, kbs, kR[0], vR, nothing);
            }
        }
        if (has_last) {
            // The last entry as a block of its own: every K row of the block is that entry (the
            // rows past it are masked), V rows past it are zero.
            Raw<KVT> kx[2][NKC], vx[NVL];
            if constexpr (KL) {
    #pragma unroll
                for (int i = 0; i < NVL; i++) kx[i / NKC][i % NKC].load(&lrow[w][0][8 * (lane % VLR)]);
            } else {
    #pragma unroll
                for (int c2 = 0; c2 < NKC; c2++) {
                    kx[0][c2].load(&lrow[w][0][32 * c2 + 8 * g]);
                    kx[1][c2] = kx[0][c2];
                }
            }
            vx[0].load(&lrow[w][1][8 * (lane % VLR)]);
            if (lane >= VLR) vx[0].set(float4{0.0f, 0.0f, 0.0f, 0.0f}, float4{0.0f, 0.0f, 0.0f, 0.0f});
    #pragma unroll
            for (int i = 1; i < NVL; i++) vx[i].set(float4{0.0f, 0.0f, 0.0f, 0.0f}, float4{0.0f, 0.0f, 0.0f, 0.0f});
            compute_block(last, I.len, kx, vx, nothing);
        }
    };
    stream();
    if constexpr (RUNS) {
        if (I.nchunk > 1) {
            // The run's state: its chunks folded left to right from a cleared state, with
            // attn_row_fold's expressions (a run's fold there, when each chunk is a unit).
            float Mr = -INFINITY, Lr = 0.0f;
            f32x4 Or[NDT];
#pragma unroll
            for (int dt = 0; dt < NDT; dt++) Or[dt] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
            auto merge_chunk = [&]() {
                float a, b, mn;
                merge_coef(Mr, m, a, b, mn);
                Lr = Lr * a + l * b;
#pragma unroll
                for (int dt = 0; dt < NDT; dt++)
#pragma unroll
                    for (int i = 0; i < 4; i++) Or[dt][i] = Or[dt][i] * a + o[dt][i] * b;
                Mr = mn;
            };
            merge_chunk();
            for (uint32_t c = cfirst + 1; c < cend; c++) {
                set_chunk(c);
                first_loads();
#pragma unroll
                for (int dt = 0; dt < NDT; dt++) o[dt] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
                m = -INFINITY;
                l = 0.0f;
                stream();
                merge_chunk();
            }
#pragma unroll
            for (int dt = 0; dt < NDT; dt++) o[dt] = Or[dt];
            m = Mr;
            l = Lr;
        }
    }
    if (!valid) return;
    if (I.nchunk == 1) {
        float* orow = p.out + ((size_t)I.row * p.nh + kvh * G + n) * hd;
#pragma unroll
        for (int dt = 0; dt < NDT; dt++) {
            const uint32_t d = 16 * dt + 4 * g;
            if (d < hd) *(float4*)(orow + d) = float4{o[dt][0] / l, o[dt][1] / l, o[dt][2] / l, o[dt][3] / l};
        }
    } else {
        // State at the canonical index of (item, KV head, chunk or run): a list's states are
        // contiguous for the fold.
        const uint32_t nst = RUNS ? (I.nchunk + ROW_RUN - 1) / ROW_RUN : I.nchunk;
        const size_t at = ((size_t)I.unit0 + (size_t)kvh * nst + uu) * 16 + n;
#pragma unroll
        for (int dt = 0; dt < NDT; dt++) {
            const uint32_t d = 16 * dt + 4 * g;
            if (d < hd) *(float4*)(p.part_o + at * HD + d) = float4{o[dt][0], o[dt][1], o[dt][2], o[dt][3]};
        }
        if (g == 0) *(float2*)(p.part_ml + at * 2) = float2{m, l};
    }
}

// One state folded into another: (M, L, O) <- fold((M, L, O), (m2, l2, o2)), four dims.
__device__ __forceinline__ void merge_state(float& M, float& L, float4& O, float m2, float l2, float4 o2) {
    float a, bb, mn;
    merge_coef(M, m2, a, bb, mn);
    L = L * a + l2 * bb;
    O = float4{O.x * a + o2.x * bb, O.y * a + o2.y * bb, O.z * a + o2.z * bb, O.w * a + o2.w * bb};
    M = mn;
}

// The fold of a one-row list's chunk states: a workgroup of ROW_FOLD_THREADS per (item, KV
// head, slot, ROW_FOLD_DIMS dims), so the loads spread over many CUs. The chunks go in runs
// of ROW_RUN consecutive chunks, each run folded left to right from a cleared state: here,
// or (p.runs) by the decode wave that streamed the run, whose states are then run states.
// R thread subsets of ROW_FOLD_DIMS / 4 threads (four dims each): subset r folds runs r,
// r + R, ... in that order from a cleared state (all its loads issued before the first
// use), then the R subset states merge as a binary tree (r with r + 1, then r with r + 2,
// ...) and the root is normalised. The order is fixed by the chunk count and the shape
// alone.
constexpr int ROW_FOLD_THREADS = 256;
constexpr int ROW_FOLD_DIMS = 32;

template <int HD>
__global__ __launch_bounds__(ROW_FOLD_THREADS) void attn_row_fold(const DirectParams p) {
    constexpr uint32_t D4 = ROW_FOLD_DIMS / 4;                          // threads per subset: 4 dims each
    constexpr uint32_t R = ROW_FOLD_THREADS / D4;                       // subsets
    constexpr uint32_t NRS = (ROW_MAX_CHUNKS / ROW_RUN + R - 1) / R;    // runs per subset at most
    constexpr uint32_t NPT = NRS * ROW_RUN;                             // chunk states per subset at most
    constexpr uint32_t NDS = (HD + ROW_FOLD_DIMS - 1) / ROW_FOLD_DIMS;  // dim slices
    static_assert(ROW_MAX_CHUNKS % ROW_RUN == 0, "whole runs");
    __shared__ float4 rO[ROW_FOLD_THREADS / 64][D4];
    __shared__ float2 rML[ROW_FOLD_THREADS / 64][D4];
    // The arguments are read before any branch on them (their scalar loads go out together);
    // a launch of one item needs no indexed read of the item.
    const uint32_t nitems = p.nitems, nkv = p.nkv, G = p.G, runs = p.runs;
    Item I = p.items[0];
    asm volatile("" ::"s"(nitems), "s"(nkv), "s"(G), "s"(runs), "s"(I.row), "s"(I.unit0), "s"(I.nchunk), "s"(p.hd),
                 "s"(p.nh), "s"(p.fuse), "s"(p.out), "s"(p.part_o), "s"(p.part_ml), "s"(p.qw), "s"(p.qrot));
    const uint32_t b = blockIdx.x / NDS, ds = blockIdx.x % NDS, per_item = nkv * G;
    const uint32_t item = b / per_item;
    if (nitems > 1) I = p.items[item];
    const uint32_t nch = I.nchunk, nrun = (nch + ROW_RUN - 1) / ROW_RUN;
    if (nch <= 1) return;  // written by the decode kernel
    const uint32_t kvh = (b % per_item) / p.G, s = (b % per_item) % p.G;
    const uint32_t tid = threadIdx.x, r = tid / D4, d = ds * ROW_FOLD_DIMS + 4 * (tid % D4);
    const size_t st0 = (size_t)I.unit0 + (size_t)kvh * (runs ? nrun : nch);  // the list's first state
    // State j of this subset's run q (run r + q R): its chunk j, or with runs the run's state
    // at j = 0.
    float2 ml[NPT];
    float4 ov[NPT];
    if (runs) {
#pragma unroll
        for (uint32_t q = 0; q < NRS; q++) {
            const uint32_t run = r + q * R;
            const size_t at = (st0 + (run < nrun ? run : 0u)) * 16 + s;
            ml[q * ROW_RUN] = *(const float2*)(p.part_ml + at * 2);
            ov[q * ROW_RUN] = *(const float4*)(p.part_o + at * HD + d);
        }
    } else {
#pragma unroll
        for (uint32_t q = 0; q < NPT; q++) {
            const uint32_t c = (r + q / ROW_RUN * R) * ROW_RUN + q % ROW_RUN;
            const size_t at = (st0 + (c < nch ? c : 0u)) * 16 + s;
            ml[q] = *(const float2*)(p.part_ml + at * 2);
            ov[q] = *(const float4*)(p.part_o + at * HD + d);
        }
    }
    // After the state loads are out (a store before them would hold them behind its load).
    if (p.fuse && tid < ROW_FOLD_DIMS && ds * ROW_FOLD_DIMS + tid < p.hd) {
        // A fused step: every unit has read q; leave head kvh * G + s rotated.
        const size_t h = (size_t)kvh * p.G + s, e = ds * ROW_FOLD_DIMS + tid;
        p.qw[((size_t)I.row * p.nh + h) * p.hd + e] = p.qrot[((size_t)item * p.nh + h) * p.hd + e];
    }
    float M = -INFINITY, L = 0.0f;
    float4 O = float4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (uint32_t q = 0; q < NRS; q++) {
        const uint32_t run = r + q * R;
        if (run < nrun) {
            float Mq = ml[q * ROW_RUN].x, Lq = ml[q * ROW_RUN].y;
            float4 Oq = ov[q * ROW_RUN];
            if (!runs) {
                Mq = -INFINITY;
                Lq = 0.0f;
                Oq = float4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
                for (uint32_t j = 0; j < ROW_RUN; j++)
                    if (run * ROW_RUN + j < nch)
                        merge_state(Mq, Lq, Oq, ml[q * ROW_RUN + j].x, ml[q * ROW_RUN + j].y, ov[q * ROW_RUN + j]);
            }
            merge_state(M, L, O, Mq, Lq, Oq);
        }
    }
    // The binary tree over the subsets (r with r + 1, then r with r + 2, ...): its levels
    // within a wave (eight subsets of D4 lanes: partners 8, 16 and 32 lanes up) by cross-lane
    // moves, without a barrier; the two across the workgroup's waves through LDS. A lane
    // whose subset is not a left operand at a level computes a value no one reads.
    auto merge = [&](float m2, float l2, float4 o2) { merge_state(M, L, O, m2, l2, o2); };
    static_assert(D4 == 8 && ROW_FOLD_THREADS == 256, "eight subsets a wave, four waves");
    {
        // partner 8 lanes up: DPP rotation by 8 within each row of 16 lanes
        auto up8 = [](float x) {
            return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x128, 0xf, 0xf, false));
        };
        merge(up8(M), up8(L), float4{up8(O.x), up8(O.y), up8(O.z), up8(O.w)});
        // partners 16 and 32 lanes up: the upper value of a permlane swap's pair
        auto up16 = [](float x) {
            return __uint_as_float(__builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false)[1]);
        };
        merge(up16(M), up16(L), float4{up16(O.x), up16(O.y), up16(O.z), up16(O.w)});
        auto up32 = [](float x) {
            return __uint_as_float(__builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false)[1]);
        };
        merge(up32(M), up32(L), float4{up32(O.x), up32(O.y), up32(O.z), up32(O.w)});
    }
    const uint32_t wv = tid / 64, q = tid % 64;  // wave; subset 8 wv holds the wave's state in lanes q < D4
    if (q < D4) {
        rO[wv][q] = O;
        rML[wv][q] = float2{M, L};
    }
    __syncthreads();
    if (q < D4 && wv % 2 == 0) {
        const float2 o2 = rML[wv + 1][q];
        merge(o2.x, o2.y, rO[wv + 1][q]);
        rO[wv][q] = O;
        rML[wv][q] = float2{M, L};
    }
    __syncthreads();
    if (q < D4 && wv == 0) {
        const float2 o2 = rML[2][q];
        merge(o2.x, o2.y, rO[2][q]);
    }
    if (r == 0 && d < p.hd)
        *(float4*)(p.out + ((size_t)I.row * p.nh + kvh * p.G + s) * p.hd + d) = float4{O.x / L, O.y / L, O.z / L, O.w / L};
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
    __shared__ __attribute__((aligned(16))) f16 vt[2][BLK * v_stride(HD)];

    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int g = lane >> 4, n = lane & 15;
    // Heaviest row blocks (latest rows, longest lists) first, across KV heads.
    const uint32_t gi_launch = p.split ? blockIdx.x / p.nchunk : blockIdx.x;
    const uint32_t cs_idx = p.split ? blockIdx.x % p.nchunk : 0u;
    const uint32_t kvh = gi_launch % p.nkv;
    const uint32_t rbi = p.nrb - 1u - gi_launch / p.nkv;
    const uint32_t grp = kvh * p.nrb + rbi;  // canonical group of the partials
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
        for (int c = 0; c < HD / 32; c++) qb[t][c] = q_operand(qrow, 32 * c + 8 * g, hd, valid[t], p.sc);
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

    const KVT* zp = (const KVT*)p.zero;
    Raw<KVT> kpre[LOADS], vpre[LOADS];
    auto load_block = [&](uint32_t key0) {
#pragma unroll
        for (int i = 0; i < LOADS; i++) {
            int e = i * NTH + tid;
            int kr = e / LPR;
            uint32_t hd0 = 8 * (e % LPR);
            uint32_t k = key0 + kr;
            bool ok = k < kb1 && hd0 < hd;
            kpre[i].load(ok ? kcb + (size_t)k * kvd + hd0 : zp);
            vpre[i].load(ok ? vcb + (size_t)k * kvd + hd0 : zp);
        }
    };
    auto store_block = [&](int stage) {
#pragma unroll
        for (int i = 0; i < LOADS; i++) {
            int e = i * NTH + tid;
            int kr = e / LPR;
            uint32_t hd0 = 8 * (e % LPR);
            *(half8*)&kl[stage][kr * KS + hd0] = kpre[i].get();
            v_store<v_stride(HD)>(vt[stage], kr, hd0, vpre[i].get());
        }
    };

    State<HD / 16> R[NT], cs[NT];
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
        // The next block (zeros past this workgroup's range: no branch, no HBM traffic).
        load_block(key0 + BLK);
        const f16* kls = kl[stage];
        block_step<HD, NT>(
            cs, qb,
            [&](int kt, int c) { return *(const half8*)&kls[(16 * kt + n) * KS + 32 * c + 8 * g]; },
            [&](int dt, int kc) { return v_operand<v_stride(HD)>(vt[stage], dt, kc, g, n); }, key0, len);
        store_block(stage ^ 1);
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

// Left fold of chunk states, R <- fold(R, c) for c = 0, 1, ... in chunk order, from a
// cleared R: the per-element arithmetic of fold(), so a split multi-row call gives the
// bits of the unsplit one. One thread per (group, slot, 4 dims), in workgroups of one
// wave so that the few thousand threads spread over as many CUs as they fill (verify: 256
// workgroups of 64 threads ran the call 1 µs faster than 64 of 256); each pass issues the
// loads of RUN chunk states before the first fold step uses them. RUN is the smallest of
// 8, 16, 24, 32 that holds a shared call's chunks (fewer loads of clamped duplicates: 0.45
// us off the 70B verify call at 4096 slots), else 32 (one batch up to 8192 entries).
// An f32 one-row step fused with RoPE (CombineParams::fuse): the fold, which runs once every
// chunk's workgroup has read q, leaves pair pp of output head h of row r rotated, as
// k_rope_append rotates q (the same expressions, so the same bits). The long fold loads the
// pair's operands when it starts (load) and rotates and stores them once it is done (store),
// so that their round trip overlaps the fold's.
struct QPair {
    float x0, x1, f;
    uint32_t pos, a, b;
    bool rot;
};
__device__ __forceinline__ QPair combine_q_load(const CombineParams& p, uint32_t r, uint32_t h, uint32_t pp) {
    QPair q{};
    q.rot = p.fuse && rope_pair(pp, p.rope_dim, p.neox, q.a, q.b);
    if (q.rot) {
        const float* qh = p.qw + ((size_t)r * p.nh + h) * p.hd;
        q.x0 = qh[q.a];
        q.x1 = qh[q.b];
        q.f = p.inv_freq[pp];
        q.pos = p.positions[r];
    }
    return q;
}
__device__ __forceinline__ void combine_q_store(const CombineParams& p, uint32_t r, uint32_t h, const QPair& q) {
    if (!q.rot) return;
    float* qh = p.qw + ((size_t)r * p.nh + h) * p.hd;
    float y0, y1;
    rotate(q.x0, q.x1, (float)q.pos * q.f, y0, y1);
    qh[q.a] = y0;
    qh[q.b] = y1;
}

constexpr int CMB_RUN = 32;

constexpr int CMB_THREADS = 64;

template <int HD, int RUN>
__global__ __launch_bounds__(CMB_THREADS) void attn_combine(const CombineParams p) {
    // The arguments are read before any branch on them, so that their scalar loads go out
    // together (one round trip to memory rather than one per branch).
    const uint32_t hd = p.hd, slots_out = p.slots_out, ngroups = p.ngroups, shared = p.shared, nrb = p.nrb,
                   rb = p.rb, G = p.G, rows = p.rows, nch_s = p.nchunk, nkv = p.nkv;
    asm volatile("" ::"s"(hd), "s"(slots_out), "s"(ngroups), "s"(shared), "s"(nrb), "s"(rb), "s"(G), "s"(rows),
                 "s"(nch_s), "s"(nkv), "s"(p.nh), "s"(p.slots), "s"(p.out), "s"(p.part_o), "s"(p.part_ml));
    const uint32_t nd4 = hd / 4;
    const uint32_t t = blockIdx.x * CMB_THREADS + threadIdx.x;
    const uint32_t d4 = t % nd4, rest = t / nd4;
    const uint32_t slot = rest % slots_out, grp = rest / slots_out;
    if (grp >= ngroups) return;
    uint32_t unit0, nchunk, r, h, step;  // chunk c's state is unit unit0 + c * step
    if (shared) {
        const uint32_t kvh = grp / nrb, rbi = grp % nrb;
        const uint32_t gh = slot / rb, rl = slot % rb;
        r = rbi * rb + rl;
        if (gh >= G || r >= rows) return;
        h = kvh * G + gh;
        unit0 = grp * nch_s;
        nchunk = nch_s;
        step = 1;
    } else {  // decode kernel states, in (item, chunk, KV head) order
        const uint32_t item = grp / nkv, kvh = grp % nkv;
        const Item& I = p.items[item];
        if (slot / G >= I.nrows || I.nchunk == 1) return;  // one chunk: written directly
        r = I.row + slot / G;
        h = kvh * G + slot % G;
        unit0 = I.unit0 + kvh;
        nchunk = I.nchunk;
        step = nkv;
    }
    const size_t stride = p.slots;  // partial slots per unit
    float M = -INFINITY, L = 0.0f;
    float4 O = float4{0.0f, 0.0f, 0.0f, 0.0f};
    for (uint32_t cb = 0; cb < nchunk; cb += RUN) {
        float2 ml[RUN];
        float4 o[RUN];
#pragma unroll
        for (int j = 0; j < RUN; j++) {
            const uint32_t c = min(cb + j, nchunk - 1);
            const size_t at = ((size_t)unit0 + (size_t)c * step) * stride + slot;
            ml[j] = *(const float2*)(p.part_ml + at * 2);
            o[j] = *(const float4*)(p.part_o + at * HD + 4 * d4);
        }
#pragma unroll
        for (int j = 0; j < RUN; j++) {
            if (cb + j < nchunk) {
                float a, b, mn;
                merge_coef(M, ml[j].x, a, b, mn);
                L = L * a + ml[j].y * b;
                O = float4{O.x * a + o[j].x * b, O.y * a + o[j].y * b, O.z * a + o[j].z * b, O.w * a + o[j].w * b};
                M = mn;
            }
        }
    }
    *(float4*)(p.out + ((size_t)r * p.nh + h) * p.hd + 4 * d4) = float4{O.x / L, O.y / L, O.z / L, O.w / L};
    // (Here the pairs' loads measured no slower than at the start: a short fold.)
    combine_q_store(p, r, h, combine_q_load(p, r, h, 2 * d4));
    combine_q_store(p, r, h, combine_q_load(p, r, h, 2 * d4 + 1));
}

// ---------------------------------------------------------------------------------------
// Prefill kernel (f16 caches, hd 128): the shared kernel's slots and arithmetic (block_step
// per 64-entry block, chunk states folded every 192 entries), with K and V blocks copied
// HBM -> LDS by the gfx950 direct-to-LDS loads, so that no VGPR holds a block in flight.
// Each load instruction of a wave fills 1 KB of LDS in lane order: four whole cache rows,
// lane l taking row 4q + l/16 and 16-byte chunk (l % 16) ^ f(row) of it, so the LDS rows
// are XOR-swizzled by chunk: K by f = row % 16 (the sixteen rows one score operand read
// takes sit on distinct banks), V by f = 2 (row % 8) (chunk pairs stay adjacent for the
// transposing reads, and the eight rows of a 32-lane half fall on distinct banks).
constexpr int PF_CPR = 16;  // 16-byte chunks per row (hd 128 in f16)

__device__ __forceinline__ uint32_t pf_kswz(uint32_t r) { return r % 16u; }
__device__ __forceinline__ uint32_t pf_vswz(uint32_t r) { return 2u * (r % 8u); }

// s_waitcnt for "at most N vector memory operations of this wave outstanding" (gfx9
// encoding: vmcnt in bits 3:0 and 15:14; expcnt and lgkmcnt left at their maximum).
template <int N>
__device__ __forceinline__ void wait_vm() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | 0xF70);
}

// Left fold of long chunk lists (more than CMB_RUN chunks: a long decode's or tree pass's
// states, an f32 cache's split passes), one workgroup per (group, output slot). The slot's
// chunk states go to LDS a segment at a time, every load of a segment in flight at once
// (direct-to-LDS, 16 bytes a lane), where attn_combine's thread would wait for a round trip
// every CMB_RUN chunks. Chunk c's weights come from the running maximum before it, which is
// the prefix maximum of the chunk maxima (a max is exact in any order): a scan across the
// threads, then merge_coef on the serial fold's operands. The threads of 4 dims each then run
// the serial recurrence over the segment's chunks in order with attn_combine's expressions,
// so the outputs are the same bits.
constexpr int CMBL_THREADS = 256;
constexpr int CMBL_BYTES = 112 * 1024;  // LDS of one segment's states

template <int HD>
__global__ __launch_bounds__(CMBL_THREADS) void attn_combine_long(const CombineParams p) {
    constexpr uint32_t D4 = HD / 4;
    constexpr uint32_t SEGC = CMBL_BYTES / (16 * D4) < CMBL_THREADS ? CMBL_BYTES / (16 * D4) : CMBL_THREADS;  // chunks a segment
    constexpr uint32_t NLD = SEGC * D4 / CMBL_THREADS;          // loads a thread a segment
    static_assert(SEGC % 8 == 0, "the recurrence reads eight chunks a batch, 16-byte aligned");
    static_assert(NLD * CMBL_THREADS == SEGC * D4 && SEGC <= CMBL_THREADS, "a segment's loads and chunks fit the threads");
    __shared__ __attribute__((aligned(16))) float4 so[SEGC * D4];
    __shared__ __attribute__((aligned(16))) float cw[3][SEGC];  // per chunk: a, b and its sum l
    __shared__ float mls[2][CMBL_THREADS];  // the segment's chunk maxima and sums
    const uint32_t hd = p.hd, slots_out = p.slots_out, ngroups = p.ngroups, shared = p.shared, nrb = p.nrb,
                   rb = p.rb, G = p.G, rows = p.rows, nch_s = p.nchunk, nkv = p.nkv;
    const uint32_t grp = blockIdx.x / slots_out, slot = blockIdx.x % slots_out;
    if (grp >= ngroups) return;
    uint32_t unit0, nchunk, r, h, step;  // chunk c's state is unit unit0 + c * step
    if (shared) {
        const uint32_t kvh = grp / nrb, rbi = grp % nrb;
        const uint32_t gh = slot / rb, rl = slot % rb;
        r = rbi * rb + rl;
        if (gh >= G || r >= rows) return;
        h = kvh * G + gh;
        unit0 = grp * nch_s;
        nchunk = nch_s;
        step = 1;
    } else {  // decode kernel states, in (item, chunk, KV head) order
        const uint32_t item = grp / nkv, kvh = grp % nkv;
        const Item& I = p.items[item];
        if (slot / G >= I.nrows || I.nchunk == 1) return;  // one chunk: written directly
        r = I.row + slot / G;
        h = kvh * G + slot % G;
        unit0 = I.unit0 + kvh;
        nchunk = I.nchunk;
        step = nkv;
    }
    // The state index of chunk c (unit unit0 + c * step, slot `slot`) fits 32 bits: the
    // workspace could not hold 2^32 states.
    const uint32_t stride = p.slots;  // partial slots per unit
    auto state = [&](uint32_t c) { return (unit0 + c * step) * stride + slot; };
    const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const QPair qp = combine_q_load(p, r, h, tid < hd / 2 ? tid : 0u);
    typedef __attribute__((address_space(3))) void lds_t;
    // Barriers without a fence: the waits before them are explicit (a fence would wait for
    // every direct-to-LDS load in flight, the states' included).
    auto barrier = [] {
        __builtin_amdgcn_sched_barrier(0);
        __builtin_amdgcn_s_barrier();
        __builtin_amdgcn_sched_barrier(0);
    };
    float M = -INFINITY;  // wave 0: the running max before the segment
    float L = 0.0f, O = 0.0f;  // threads tid < HD: the fold of dim tid and of the sums
    for (uint32_t c0 = 0; c0 < nchunk; c0 += SEGC) {
        const uint32_t nseg = min(SEGC, nchunk - c0);
        barrier();  // wave 0 is done with the previous segment's LDS
        // Chunk c0 + 64 wave + lane's max and sum (two 4-byte loads), then the states: load i
        // of the workgroup, lane l, fills so[256 i + 64 wave + l] with 16 bytes of chunk
        // c0 + e / D4 (e that index). Chunks past the list load its last.
        {
            const float* src = p.part_ml + (size_t)state(min(c0 + 64 * wave + lane, nchunk - 1u)) * 2;
            __builtin_amdgcn_global_load_lds((const void*)src, (lds_t*)&mls[0][64 * wave], 4, 0, 0);
            __builtin_amdgcn_global_load_lds((const void*)(src + 1), (lds_t*)&mls[1][64 * wave], 4, 0, 0);
        }
        // (Load i's chunk is c0 + i * CPL + tid / D4, its dims 4 (tid % D4) .. + 3.)
        constexpr uint32_t CPL = CMBL_THREADS / D4;  // chunks a workgroup load covers
        static_assert(CMBL_THREADS % D4 == 0, "a load covers whole chunks");
        // Load i's address: the first load's plus i steps of CPL chunks (chunk states are
        // step * stride apart), or the list's last chunk's once past it.
        const float* ob = p.part_o + 4 * (tid % D4);
        const uint32_t cf = c0 + tid / D4;
        const float* a0 = ob + (size_t)state(min(cf, nchunk - 1u)) * HD;
        const float* alast = ob + (size_t)state(nchunk - 1u) * HD;
        const size_t inc = (size_t)CPL * step * stride * HD;
#pragma unroll
        for (uint32_t i = 0; i < NLD; i++) {
            const float* src = cf + i * CPL < nchunk ? a0 + i * inc : alast;
            __builtin_amdgcn_global_load_lds((const void*)src, (lds_t*)&so[i * CMBL_THREADS + 64 * wave], 16, 0, 0);
        }
        wait_vm<NLD>();  // this wave's maxima and sums are in
        barrier();       // and every wave's
        if (wave == 0) {
            // Lane l's four chunks 4l .. 4l + 3: their maxima (-inf past the segment), the
            // prefix within the four, then the wave's exclusive scan of the lanes' maxima.
            float mv[4];
#pragma unroll
            for (uint32_t j = 0; j < 4; j++) mv[j] = 4 * lane + j < nseg ? mls[0][4 * lane + j] : -INFINITY;
            const float tot = fmaxf(fmaxf(mv[0], mv[1]), fmaxf(mv[2], mv[3]));
            float inc = tot;
#pragma unroll
            for (int d = 1; d < 64; d <<= 1) {
                const float t = __shfl_up(inc, d);
                if (lane >= (uint32_t)d) inc = fmaxf(inc, t);
            }
            float run = __shfl_up(inc, 1);
            run = lane == 0 ? M : fmaxf(M, run);  // the running max before chunk 4l
#pragma unroll
            for (uint32_t j = 0; j < 4; j++) {
                const uint32_t c = 4 * lane + j;
                float a, b, mn;
                merge_coef(run, mv[j], a, b, mn);
                if (c < nseg) {
                    cw[0][c] = a;
                    cw[1][c] = b;
                    cw[2][c] = mls[1][c];
                }
                run = mn;
            }
            M = fmaxf(M, __shfl(inc, 63));
        }
        wait_vm<0>();
        barrier();  // every wave's states are in
        // Thread d < HD: dim d's recurrence. The sums' recurrence runs in the wave after the
        // dims' (every dims thread runs it as well when the dims take all four waves). Full
        // runs of 32 chunks are straight-line code, so the compiler issues their LDS reads
        // ahead of the steps that take them; then runs of 8, then single chunks.
        const float* sof = (const float*)so;
        constexpr bool SPARE = HD < CMBL_THREADS;  // a wave past the dims computes the sums
        const bool dims = tid < (uint32_t)HD, sums = SPARE ? (tid >= (uint32_t)HD && tid < (uint32_t)HD + 64u) : dims;
        auto run = [&](uint32_t c, auto N) {
            constexpr uint32_t n = decltype(N)::value;
            if (dims) {
#pragma unroll
                for (uint32_t j = 0; j < n; j++) O = O * cw[0][c + j] + sof[(c + j) * HD + tid] * cw[1][c + j];
            }
            if (sums) {
#pragma unroll
                for (uint32_t j = 0; j < n; j++) L = L * cw[0][c + j] + cw[2][c + j] * cw[1][c + j];
            }
        };
        uint32_t c = 0;
        for (; c + 32 <= nseg; c += 32) run(c, std::integral_constant<uint32_t, 32>{});
        for (; c + 8 <= nseg; c += 8) run(c, std::integral_constant<uint32_t, 8>{});
        for (; c < nseg; c++) run(c, std::integral_constant<uint32_t, 1>{});
    }
    // The sums' lane hands L to the dims.
    __shared__ float lfin;
    if constexpr (HD < CMBL_THREADS) {
        if (tid == (uint32_t)HD) lfin = L;
        __syncthreads();
        L = lfin;
    }
    if (tid < hd) p.out[((size_t)r * p.nh + h) * hd + tid] = O / L;
    if (tid < hd / 2) combine_q_store(p, r, h, qp);
}

// V^T tiles of a prefill call (written by vt_pack): per KV head, hd rows of npad keys, each
// 32-key group stored in the order the PV operand takes it (lane group g holds keys
// 4g..4g+3 and 16+4g..16+4g+3), so that a lane's eight keys of one dim are 16 contiguous
// bytes: V^T operands are plain 16-byte LDS reads instead of transposing ones.
__device__ __forceinline__ uint32_t vt_pos(uint32_t q) {  // key q of a 32-group -> position
    return 8 * ((q & 15) >> 2) + 4 * (q >> 4) + (q & 3);
}

__global__ __launch_bounds__(256) void vt_pack(const f16* __restrict__ vc, f16* __restrict__ vt, uint32_t kvd,
                                               uint32_t nkeys, uint32_t npad) {
    constexpr int HD = 128, TS = HD + 2;
    __shared__ f16 tile[64 * TS];
    const uint32_t kvh = blockIdx.y, key0 = blockIdx.x * 64, tid = threadIdx.x;
    // 64 keys x 128 dims in, rows past the list as zeros.
    for (uint32_t e = tid; e < 64 * (HD / 8); e += 256) {
        const uint32_t r = e / (HD / 8), c = 8 * (e % (HD / 8)), key = key0 + r;
        half8 v = half8{0, 0, 0, 0, 0, 0, 0, 0};
        if (key < nkeys) v = *(const half8*)(vc + (size_t)key * kvd + (size_t)kvh * HD + c);
#pragma unroll
        for (int j = 0; j < 8; j++) tile[r * TS + c + j] = v[j];
    }
    __syncthreads();
    // hd rows of 64 positions out: 8 positions (16 bytes) a thread per step.
    for (uint32_t e = tid; e < HD * 8; e += 256) {
        const uint32_t d = e / 8, p0 = 8 * (e % 8);
        half8 v;
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const uint32_t pos = p0 + j, b = pos / 32, pq = pos % 32;
            const uint32_t q = 4 * (pq / 8) + 16 * ((pq % 8) / 4) + (pq % 4);  // inverse of vt_pos
            v[j] = tile[(32 * b + q) * TS + d];
        }
        *(half8*)(vt + ((size_t)kvh * HD + d) * npad + key0 + p0) = v;
    }
}

// The softmax of a 16-slot tile over a 64-entry block (block_step's): scores in log2 units
// -> the P^T operands pb (f16) and the tile's new max and sum; corr is the factor its O takes
// before the block's PV.
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
template <int NDT>
__device__ __forceinline__ void tile_softmax(State<NDT>& s, const f32x4 (&x)[4], half8 (&pb)[2], float& corr) {
    float mx = fmaxf(fmaxf(x[0][0], x[0][1]), fmaxf(x[0][2], x[0][3]));
#pragma unroll
    for (int kt = 1; kt < 4; kt++) mx = fmaxf(mx, fmaxf(fmaxf(x[kt][0], x[kt][1]), fmaxf(x[kt][2], x[kt][3])));
    mx = tile_max(mx);
    float mn, ms;
    lazy_max(s.m, mx, mn, ms, corr);
    // P in f16 once: the block sum (dot2 chain over the pairs, tiles in order, then across
    // lanes) and the PV operand (keys 32kc + 4g + 0..3, then 32kc + 16 + 4g + 0..3).
    uint32_t hp[4][2];
    float ls = 0.0f;
#pragma unroll
    for (int kt = 0; kt < 4; kt++)
#pragma unroll
        for (int j = 0; j < 2; j++) {
            const half2 h = half2{(f16)exp2_hw(x[kt][2 * j] - ms), (f16)exp2_hw(x[kt][2 * j + 1] - ms)};
            ls = pair_sum(h, ls);
            hp[kt][j] = __builtin_bit_cast(uint32_t, h);
        }
    const float ps = tile_sum(ls);
    s.l = s.l * corr + ps;
    s.m = mn;
#pragma unroll
    for (int kc = 0; kc < 2; kc++)
        pb[kc] = __builtin_bit_cast(half8, u32x4{hp[2 * kc][0], hp[2 * kc][1], hp[2 * kc + 1][0], hp[2 * kc + 1][1]});
}

// ---------------------------------------------------------------------------------------
// Single-launch fold of split chunks (group fold). A split launch's workgroups of one group
// (one KV head's row block) each compute one chunk's state. Instead of a second kernel
// (attn_combine) that starts once the whole launch has drained, every workgroup publishes its
// state, counts itself in at the group's arrival counter, waits until the group's nchunk
// workgroups are all in, and then folds one slice of the group's outputs over all the chunks:
// the same left fold, in chunk order, with attn_combine's expressions, so the outputs are the
// same bits.
// Where the states travel: each XCD has its own L2, and another XCD sees a plain store only
// after that L2 is written back. The launch places a group's workgroups on one XCD when it
// can (workgroups go to the XCDs in turn, so block indices 8 apart share one), and each
// workgroup records the XCD it runs on (its XCC_ID) in the group's mask. A group found on one
// XCD exchanges its states through that XCD's L2: plain stores, plain loads. A group spread
// over several (a different dispatch order, a device in another partition mode) publishes
// every state again with write-through stores, counts in a second time, and reads them after
// an agent-scope acquire; its results are the same bits, only later.
// The host takes this path only when every workgroup of the launch can be resident at once
// (one a CU, at most as many as the device has CUs), so a waiting workgroup never holds a CU
// that another of its group needs. The waits are bounded all the same: if other work holds
// the GPU past the bound, the workgroup stops waiting, writes NaN for its outputs and sets the
// context's error word, which bchip_sync reports.
// Per group, GROUP_STRIDE words at gcnt + grp * GROUP_STRIDE: a 64-bit arrival word (the
// count in bits 0-15, the sum of the arrivals' XCC_IDs in bits 16-31 and the sum of their
// squares in bits 32-63: one poll tells both that all are in and whether all ran on one XCD,
// as n * sum(x^2) == sum(x)^2 exactly when every x is the same), the second arrivals, and the
// departures; the last workgroup to leave clears them for the next call.
constexpr uint32_t GFOLD_MAX_CHUNKS = 32;
// Rows a fused multi-row pass takes (one row block: 64 slots of at least 4 heads a KV head).
constexpr uint32_t FUSE_ROWS = 16;
// A wait takes at most SharedParams::gspins polls (2^16 unless a test lowers it), each a
// counter read and ~128 clocks of sleep.
enum : uint32_t { GS_ARRIVE = 0, GS_ARRIVE2 = 2, GS_LEAVE = 3 };
enum : uint32_t { GF_TIMEOUT = 0, GF_LOCAL = 1, GF_SPREAD = 2 };

// A store that writes through to device memory (agent-scope coherence): once this wave's
// vmcnt has drained it is visible to agent-scope loads from any XCD, with no L2 write-back.
__device__ __forceinline__ void store_wt4(float* p, f32x4 v) {
    asm volatile("global_store_dwordx4 %0, %1, off sc1" ::"v"(p), "v"(v) : "memory");
}
__device__ __forceinline__ void store_wt2(float* p, float a, float b) {
    typedef float f32x2 __attribute__((ext_vector_type(2)));
    asm volatile("global_store_dwordx2 %0, %1, off sc1" ::"v"(p), "v"(f32x2{a, b}) : "memory");
}

// The XCD this wave runs on (HW_REG_XCC_ID, bits 3:0).
__device__ __forceinline__ uint32_t xcc_id() { return __builtin_amdgcn_s_getreg(20 | (0 << 6) | (3 << 11)); }

// A workgroup's side of its group's synchronisation, carried from the arrival to the
// departure. Thread 0 arrives and waits; the workgroup's last thread counts it out (a lane
// with no fold work at verify sizes, so that the count's round trip, which its wave's later
// loads would wait behind, holds up none of the fold's loads).
struct GroupSync {
    uint32_t* gs;
    uint32_t n;
    uint32_t spins;      // polls a wait may take
    uint32_t spread;     // take the spread path whatever the XCDs
    uint32_t leave_old;  // the last thread: the departure count before this workgroup's
};

__device__ __forceinline__ void group_depart(GroupSync& s) {
    if (threadIdx.x == blockDim.x - 1)
        s.leave_old = __hip_atomic_fetch_add(s.gs + GS_LEAVE, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Called by every thread once the workgroup's state is stored (plain stores). Returns
// GF_LOCAL (the group ran on one XCD: the states are in its L2; the workgroup has counted
// itself out, nothing later waits on the group's words), GF_SPREAD (the caller must publish
// its state again write-through and call group_second), or GF_TIMEOUT. flag: an LDS word
// the workgroup no longer uses (the kernels' LDS is full).
__device__ __forceinline__ uint32_t group_arrive(GroupSync& s, uint32_t* err, uint32_t& flag) {
    __builtin_amdgcn_s_waitcnt(0);  // this thread's stores are done
    __syncthreads();
    if (threadIdx.x == 0) {
        uint64_t* word = (uint64_t*)(s.gs + GS_ARRIVE);
        const uint64_t x = xcc_id();
        __hip_atomic_fetch_add(word, 1ull | (x << 16) | (x * x << 32), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        uint32_t mode = GF_TIMEOUT;
        uint64_t v = 0;
        for (uint32_t spins = 0;; spins++) {
            v = __hip_atomic_load(word, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            if ((uint32_t)(v & 0xffff) >= s.n || spins == s.spins) break;
            __builtin_amdgcn_s_sleep(2);
        }
        if ((uint32_t)(v & 0xffff) >= s.n) {
            const uint64_t sx = (v >> 16) & 0xffff, sxx = v >> 32;
            mode = (uint64_t)s.n * sxx == sx * sx && !s.spread ? GF_LOCAL : GF_SPREAD;
            // This CU's L1 holds nothing of other workgroups' states; drop it all the same.
            if (mode == GF_LOCAL) asm volatile("buffer_inv sc0" ::: "memory");
        } else {
            __hip_atomic_store(err, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
        }
        flag = mode;
    }
    __syncthreads();
    const uint32_t mode = flag;
    if (mode == GF_LOCAL) group_depart(s);
    return mode;
}

// A spread group, after the caller stored its state again write-through: the second count,
// the departure, then an agent-scope acquire (this CU's L1 and this XCD's L2 drop what they
// hold of other XCDs' writes). Returns GF_SPREAD or GF_TIMEOUT.
__device__ __forceinline__ uint32_t group_second(GroupSync& s, uint32_t* err, uint32_t& flag) {
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (threadIdx.x == 0) {
        uint32_t* w = s.gs + GS_ARRIVE2;
        __hip_atomic_fetch_add(w, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        uint32_t spins = 0;
        while (__hip_atomic_load(w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) < s.n && ++spins < s.spins)
            __builtin_amdgcn_s_sleep(2);
        const bool ok = spins < s.spins;
        if (!ok) __hip_atomic_store(err, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
        flag = ok ? GF_SPREAD : GF_TIMEOUT;
    }
    __syncthreads();
    const uint32_t mode = flag;
    if (mode == GF_SPREAD) group_depart(s);
    return mode;
}

// Thread 0 of the last workgroup to have counted itself out clears the group's words for the
// next call (every workgroup of the group had passed every wait when it counted out).
__device__ __forceinline__ void group_leave(const GroupSync& s) {
    if (threadIdx.x == blockDim.x - 1 && s.leave_old == s.n - 1) {
#pragma unroll
        for (uint32_t i = 0; i < 4; i++) __hip_atomic_store(s.gs + i, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}

// Workgroup cs_idx's share of group grp's outputs: slots cs_idx * per .. (per = SL / nchunk,
// rounded up), one slot a wave at a time, two dims a lane. Each output is attn_combine's fold
// over the group's chunk states in chunk order. Its weights depend only on the running maxima,
// which are the prefix maxima of the chunks' maxima (a max is exact in any order): lane c
// takes chunk c's max and sum, a scan across lanes gives the maximum of the chunks before it,
// and lane c computes chunk c's pair of weights from the same operands as the serial fold.
// The sum and the two dims then run the serial recurrence, every lane reading each chunk's
// weights and sum back from LDS (wts: GFOLD_MAX_CHUNKS float4 a wave, LDS the workgroup no
// longer uses), so every product and sum is the serial fold's, in its order.
template <int SL>
__device__ __forceinline__ void group_fold_slots(const SharedParams& p, uint32_t grp, uint32_t cs_idx, uint32_t rbi,
                                                 uint32_t kvh, bool ok, float4* wts) {
    constexpr uint32_t HD = 128, MC = GFOLD_MAX_CHUNKS;
    static_assert(MC <= 32, "a chunk's weights sit in lanes 0..31");
    const uint32_t nch = p.nchunk;
    const uint32_t lane = threadIdx.x & 63;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), nw = blockDim.x >> 6;
    const uint32_t per = (SL + nch - 1) / nch;
    const uint32_t lo = cs_idx * per, hi = min(lo + per, (uint32_t)SL);
    for (uint32_t slot = lo + wave; slot < hi; slot += nw) {
        const uint32_t gh = slot / p.rb, r = rbi * p.rb + slot % p.rb;
        if (gh >= p.G || r >= p.rows) continue;
        float* dst = p.out + ((size_t)r * p.nh + kvh * p.G + gh) * HD + 2 * lane;
        if (!ok) {
            const float qnan = __uint_as_float(0x7fc00000u);  // a bit pattern: this object has no NaN arithmetic
            *(float2*)dst = float2{qnan, qnan};
            continue;
        }
        // The states of a group fold sit as [group][slot][chunk][HD], a slot's chunks 512 bytes
        // apart, and the workspace holds GFOLD_MAX_CHUNKS chunk states past the last group's:
        // every load is unconditional and off one base (chunks past the group's last read
        // whatever follows, unused). A load behind a branch would make the compiler wait for
        // all loads in flight where it joins.
        const size_t sbase = ((size_t)grp * SL + slot) * nch;
        const float2 ml = *(const float2*)(p.part_ml + (sbase + (lane & (MC - 1))) * 2);
        const float* ob = p.part_o + sbase * HD + 2 * lane;
        float2 o[MC];
#pragma unroll
        for (uint32_t c = 0; c < MC; c++) o[c] = *(const float2*)(ob + c * HD);
        const float mc = lane < nch ? ml.x : -INFINITY;
        // Inclusive prefix max over lanes 0..31 by DPP moves (a lane whose source falls
        // outside the pattern takes -inf, the max's identity): shifts right by 1, 2, 4 and 8
        // within each row of 16 lanes, then lane 15's max broadcast into row 1; then the
        // whole wave shifted right by one lane, so lane c holds the max of chunks 0..c-1.
        auto dpp = [](float x, auto ctrl, auto rows) {
            return __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(-INFINITY), __float_as_int(x),
                                                               decltype(ctrl)::value, decltype(rows)::value, 0xf, false));
        };
        float pm = mc;
        pm = fmaxf(pm, dpp(pm, std::integral_constant<int, 0x111>{}, std::integral_constant<int, 0xf>{}));  // row_shr:1
        pm = fmaxf(pm, dpp(pm, std::integral_constant<int, 0x112>{}, std::integral_constant<int, 0xf>{}));  // row_shr:2
        pm = fmaxf(pm, dpp(pm, std::integral_constant<int, 0x114>{}, std::integral_constant<int, 0xf>{}));  // row_shr:4
        pm = fmaxf(pm, dpp(pm, std::integral_constant<int, 0x118>{}, std::integral_constant<int, 0xf>{}));  // row_shr:8
        pm = fmaxf(pm, dpp(pm, std::integral_constant<int, 0x142>{}, std::integral_constant<int, 0xa>{}));  // row_bcast:15
        const float before = dpp(pm, std::integral_constant<int, 0x138>{}, std::integral_constant<int, 0xf>{});  // wave_shr:1
        float a, b, mn;
        merge_coef(before, mc, a, b, mn);
        float4* wl = wts + wave * MC;
        if (lane < MC) wl[lane] = float4{a, b, ml.y, 0.0f};
        float L = 0.0f, O0 = 0.0f, O1 = 0.0f;
        // Eight chunks' weights a read batch (one address for the whole wave: broadcast
        // reads), then eight steps, each a uniform branch the compiler keeps.
#pragma unroll
        for (uint32_t c0 = 0; c0 < MC; c0 += 8) {
            if (c0 >= nch) break;
            float4 wc[8];
#pragma unroll
            for (uint32_t j = 0; j < 8; j++) wc[j] = wl[c0 + j];
#pragma unroll
            for (uint32_t j = 0; j < 8; j++) {
                if (c0 + j < nch) {
                    keep_branch();
                    L = L * wc[j].x + wc[j].z * wc[j].y;
                    O0 = O0 * wc[j].x + o[c0 + j].x * wc[j].y;
                    O1 = O1 * wc[j].x + o[c0 + j].y * wc[j].y;
                }
            }
        }
        *(float2*)dst = float2{O0 / L, O1 / L};
    }
}

// The prefill kernel proper: one 16-slot tile per wave, W waves sharing each K and V block
// in LDS, block_step's arithmetic per slot. Blocks stream through a ring of three LDS
// stages (one LDS object each, K then V), one chunk's worth, fetched two blocks ahead by
// direct-to-LDS loads, with one barrier per block. The loop is unrolled by the chunk, so
// that every stage is a compile-time object (the compiler then waits for a stage's own
// loads before reading it, not for every load in flight) and the chunk fold sits in
// straight-line code between chunks (measured against a four-stage ring with the fold
// behind a branch: 505 / 640 TFLOP/s at 2048 / 8192 rows against 491 / 625, and verify
// 11.9 µs against 14.0 at 4096 slots).
// Not kept (measured slower): two tiles a wave at one wave a SIMD (each V operand read
// once for two MFMAs, one tile's softmax scheduled beside the other's MFMAs, R in LDS):
// 370 / 460 TFLOP/s; raising a wave's priority over its MFMAs: 3-7% slower.
// The per-block work is cut to what the arithmetic needs:
//  - rows are fetched from per-lane offsets fixed for the whole loop plus a scalar block
//    base; only a block that ends past the list selects the zero page per lane, and nothing
//    past the list is fetched;
//  - the mask test is one vote per tile; LDS operand reads are per-lane bases plus
//    immediate offsets;
//  - P is rounded to f16 once, for both the block sum and the PV operand.
template <int N>
using ic = std::integral_constant<int, N>;

template <int W, bool VT, bool FUSE>
__global__ __launch_bounds__(64 * W) void attn_prefill(const SharedParams p) {
    constexpr int HD = 128;
    constexpr int NKC = HD / 32, NDT = HD / 16;
    constexpr int STAGES = CHUNK_MULTI / BLK;   // ring stages: one chunk
    constexpr int RPI = 64 / PF_CPR;            // cache rows per load instruction
    constexpr int LPW = BLK / RPI / W;          // load instructions per wave per block (K or V)
    constexpr int LPB = 2 * LPW;                // K and V loads per wave per block
    constexpr int SZ = 2 * BLK * HD;            // f16 per stage: K rows, then V (or V^T)
    static_assert(LPW * RPI * W == BLK, "a block's rows divide over the waves");
    static_assert(STAGES == 3 && CHUNK_MULTI % BLK == 0, "the loop below is unrolled by three blocks");
    __shared__ __attribute__((aligned(16))) f16 ring0[SZ];
    __shared__ __attribute__((aligned(16))) f16 ring1[SZ];
    __shared__ __attribute__((aligned(16))) f16 ring2[SZ];
    // Each wave's Q tile as loaded: 2 * NKC rows of 64 lanes x 4 floats.
    __shared__ __attribute__((aligned(16))) float qlds[W][2 * NKC * 256];
    // FUSE: the rotations' sines and cosines, row rl of the workgroup and pair pp at
    // rsc[64 rl + pp] (hd 128: 64 pairs); after the blocks, the group fold's flag word.
    __shared__ float2 rsc[FUSE ? FUSE_ROWS * 64 : 1];
    // FUSE: the launch's new rows of this KV head as the cache holds them, K rotated: [row][hd].
    __shared__ __attribute__((aligned(16))) f16 nrow[FUSE ? 2 : 1][FUSE ? FUSE_ROWS * HD : 8];
    // FUSE: each wave's copy of the rotation frequencies (pair pp), loaded direct to LDS.
    __shared__ __attribute__((aligned(16))) float sfreq[FUSE ? W : 1][64];
    auto ring = [&](auto S) -> f16* {
        if constexpr (decltype(S)::value == 0) return ring0;
        else if constexpr (decltype(S)::value == 1) return ring1;
        else return ring2;
    };

    const int tid = threadIdx.x, lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int g = lane >> 4, n = lane & 15;
    // Split launches: block -> (group in launch order, chunk). With xmap, blocks 8 apart (one
    // XCD's share when workgroups go to the XCDs in turn) take one group's chunks.
    uint32_t gi_launch = blockIdx.x, cs_idx = 0;
    if (p.split) {
        if (p.xmap) {
            const uint32_t x = blockIdx.x % 8u, k = blockIdx.x / 8u;
            gi_launch = x + 8u * (k / p.nchunk);
            cs_idx = k % p.nchunk;
        } else {
            gi_launch = blockIdx.x / p.nchunk;
            cs_idx = blockIdx.x % p.nchunk;
        }
    }
    const uint32_t kvh = gi_launch % p.nkv;
    const uint32_t rbi = p.nrb - 1u - gi_launch / p.nkv;  // heaviest row blocks first
    const uint32_t grp = kvh * p.nrb + rbi;
    const uint32_t r0 = rbi * p.rb;
    const uint32_t rlast = min(r0 + p.rb, p.rows) - 1u;
    const uint32_t maxlen = p.pos + rlast + 1u;
    const uint32_t kvd = p.nkv * HD;

    // Slot n of this wave is slot 16w + n of the workgroup: head gh, row r0 + rl. Its Q is
    // loaded here and converted after the first K/V loads are issued, so that the two
    // latencies overlap.
    half8 qb[NKC];
    uint32_t len, orow, ohead;
    bool valid;
    {
        const uint32_t sl = 16 * w + n;
        const uint32_t gh = sl / p.rb, rl = sl % p.rb, r = r0 + rl;
        valid = gh < p.G && r < p.rows;
        len = valid ? p.pos + r + 1u : 0u;
        orow = r;
        ohead = kvh * p.G + gh;
        const float* qrow = valid ? p.q + ((size_t)r * p.nh + ohead) * HD : (const float*)p.zero;
        // Q goes to the wave's own LDS rows by direct-to-LDS loads, each lane's 16 bytes to
        // its own place, like the blocks after it: the compiler counts a wait for them per
        // LDS object, so the conversion below waits for Q alone, not for the blocks issued
        // after it (loads into registers would be counted as the last ones issued).
        typedef __attribute__((address_space(3))) void lds_q_t;
        if constexpr (FUSE) {
            // FUSE: first this wave's copy of the rotation frequencies (pair pp = lane; pairs
            // past rope_dim / 2 read the zero page), so that the table can go before Q lands.
            __builtin_amdgcn_global_load_lds(
                (const void*)((uint32_t)lane < p.rope_dim / 2 ? p.inv_freq + lane : (const float*)p.zero),
                (lds_q_t*)&sfreq[w][0], 4, 0, 0);
        }
#pragma unroll
        for (int c = 0; c < NKC; c++) {
            const float* src = valid ? qrow + 32 * c + 8 * g : qrow;
            __builtin_amdgcn_global_load_lds((const void*)src, (lds_q_t*)&qlds[w][(2 * c) * 256], 16, 0, 0);
            __builtin_amdgcn_global_load_lds((const void*)(src + 4), (lds_q_t*)&qlds[w][(2 * c + 1) * 256], 16, 0, 0);
        }
    }
    uint32_t kb0, kb1;
    if (p.split) {
        kb0 = cs_idx * CHUNK_MULTI;
        kb1 = min(kb0 + CHUNK_MULTI, maxlen);
    } else {
        kb0 = 0;
        kb1 = maxlen;
    }

    // Per-lane element offsets of this wave's load instructions, fixed for the loop: K row
    // 4q + l/16 (q = i*W + w), 16-byte chunk l%16 swizzled by the row; V^T dim row 8q + l/8,
    // chunk l%8 swizzled by the dim row (VT), else V rows as K.
    // FUSE: the small loads go direct to LDS before the blocks' (a wave's loads complete in
    // issue order, and loads into registers would make the compiler wait for every load in
    // flight before their first use): the frequencies (above, before Q), and, for a chunk that
    // holds new rows, the rows of k and v of this KV head (f32, [row][hd]) into the third ring
    // stage, which the blocks reach only after the prologue. Rows past the launch's read the
    // zero page.
    typedef __attribute__((address_space(3))) void lds_f_t;
    const bool has_new = FUSE && kb1 > p.pos;
    float* raw = (float*)ring2;  // FUSE: k rows at raw[r * HD], v rows at raw[FUSE_ROWS * HD + r * HD]
    if constexpr (FUSE) {
        const float* zf = (const float*)p.zero;
        if (has_new) {
#pragma unroll
            for (int i = 0; i < 2; i++) {
                const uint32_t c = (2 * w + i) * 64 + lane, r = c / 32, d = 4 * (c % 32);  // 16-byte pieces
                const bool ok = r < p.rows;
                const size_t at = ((size_t)r * p.nkv + kvh) * HD + d;
                __builtin_amdgcn_global_load_lds((const void*)(ok ? p.knew + at : zf), (lds_f_t*)&raw[(2 * w + i) * 256], 16, 0, 0);
                __builtin_amdgcn_global_load_lds((const void*)(ok ? p.vnew + at : zf),
                                                 (lds_f_t*)&raw[FUSE_ROWS * HD + (2 * w + i) * 256], 16, 0, 0);
            }
        }
    }
    const f16* zp = (const f16*)p.zero;
    const f16* kcb = (const f16*)p.kc + (size_t)kvh * HD;
    const f16* vcb = VT ? (const f16*)p.vt + (size_t)kvh * HD * p.vt_npad : (const f16*)p.vc + (size_t)kvh * HD;
    uint32_t krow[LPW], koff[LPW], voff[LPW];
#pragma unroll
    for (int i = 0; i < LPW; i++) {
        const uint32_t q = i * W + w, row = q * RPI + lane / PF_CPR, pch = lane % PF_CPR;
        krow[i] = row;
        koff[i] = row * kvd + 8 * (pch ^ pf_kswz(row));
        if constexpr (VT) {
            const uint32_t d = q * 8 + lane / 8;
            voff[i] = d * p.vt_npad + 8 * ((lane % 8) ^ (d % 8));
        } else {
            voff[i] = row * kvd + 8 * (pch ^ pf_vswz(row));
        }
    }
    typedef __attribute__((address_space(3))) void lds_t;
    // A block within the list issues LPB loads per wave, rows past the list from the zero
    // page; a block past the list issues none.
    auto load_block = [&](uint32_t key0, auto S) {
        if (key0 >= kb1) return;  // nothing past the list
        f16* kl = ring(S);
        f16* vl = kl + BLK * HD;
        const f16* kb = kcb + (size_t)key0 * kvd;
        const f16* vb = VT ? vcb + key0 : vcb + (size_t)key0 * kvd;
        if (key0 + BLK <= kb1) {
#pragma unroll
            for (int i = 0; i < LPW; i++) {
                const uint32_t q = i * W + w;
                __builtin_amdgcn_global_load_lds((const void*)(kb + koff[i]), (lds_t*)&kl[q * RPI * HD], 16, 0, 0);
                __builtin_amdgcn_global_load_lds((const void*)(vb + voff[i]), (lds_t*)&vl[q * (VT ? 8 * BLK : RPI * HD)], 16, 0, 0);
            }
        } else {
            // The list's last block: rows past it read the zero page (the packed V^T holds
            // zeros there already).
#pragma unroll
            for (int i = 0; i < LPW; i++) {
                const uint32_t q = i * W + w;
                const bool ok = key0 + krow[i] < kb1;
                const f16* ks = ok ? kb + koff[i] : zp + 8 * (lane % PF_CPR);
                const f16* vs = (VT || ok) ? vb + voff[i] : zp + 8 * (lane % PF_CPR);
                __builtin_amdgcn_global_load_lds((const void*)ks, (lds_t*)&kl[q * RPI * HD], 16, 0, 0);
                __builtin_amdgcn_global_load_lds((const void*)vs, (lds_t*)&vl[q * (VT ? 8 * BLK : RPI * HD)], 16, 0, 0);
            }
        }
    };
    // LDS operand bases: K tile kt, hd chunk c at kbase[c] + kt * 16 rows (row 16kt + n has
    // swizzle n); V^T tile dt, key half kc at vbase[kc] + dt * 16 dim rows (swizzle n % 8).
    uint32_t kbase[NKC], vbase[2];
#pragma unroll
    for (int c = 0; c < NKC; c++) kbase[c] = n * HD + 8 * ((4 * c + g) ^ n);
#pragma unroll
    for (int kc = 0; kc < 2; kc++) vbase[kc] = n * BLK + 8 * ((4 * kc + g) ^ (n % 8));
    // The transposing V reads' lane terms: row 4g + n/4 of a 32-row half (rows r and r + 16
    // share the swizzle 2 (r % 8)), its half-chunk (n % 4) / 2 and dims half n % 2 (in f16),
    // and the 16-dim chunk swizzle.
    const uint32_t vrow = (4 * g + (n >> 2)) * HD + 8 * ((n & 3) >> 1) + 4 * (n & 1);
    const uint32_t vsw = (4 * g + (n >> 2)) % 8;
    // Barrier without the fence __syncthreads carries: that fence would wait for every
    // direct-to-LDS load in flight, the later blocks' included. The waits before it are
    // explicit; LDS reads of a wave finish before its MFMAs consume them, so every read of a
    // stage is over when its wave reaches the next barrier.
    auto barrier = [&]() {
        __builtin_amdgcn_sched_barrier(0);
        __builtin_amdgcn_s_barrier();
        __builtin_amdgcn_sched_barrier(0);
    };

    State<NDT> R, cs;
    state_clear(R);
    state_clear(cs);
    // Prologue: blocks 0 .. STAGES-2 in flight. (A workgroup of a split launch may see
    // nothing of its chunk: then it only stores its empty states.) Q waits only for its own
    // loads, which went out before the blocks' (a wave's loads complete in issue order): the
    // blocks stay in flight through the conversion. The waits count the blocks' loads
    // exactly, and the LDS reads of Q are written out, so that the compiler does not add
    // its own wait for every load in flight before them (it does not count direct-to-LDS
    // loads as younger than Q's).
    load_block(kb0, ic<0>{});
    load_block(kb0 + BLK, ic<1>{});
    // Blocks now in flight (their load instructions, this wave).
    const int inflight = kb0 + BLK < kb1 ? 2 : kb0 < kb1 ? 1 : 0;
    if constexpr (FUSE) {
        // The frequencies in (the wait leaves Q, the new rows and the blocks in flight: they went
        // out after them, in that order), then
        // the table of the rotations' sines and cosines, row rl of the workgroup and pair pp at
        // rsc[64 rl + pp], wave w taking rows w, w + W, ...
        constexpr int NQ = 2 * NKC, NR = 4;  // Q's and the new rows' load instructions, this wave
        if (has_new) {
            if (inflight == 2) wait_vm<NQ + NR + 2 * LPB>();
            else if (inflight == 1) wait_vm<NQ + NR + LPB>();
            else wait_vm<NQ + NR>();
        } else {
            if (inflight == 2) wait_vm<NQ + 2 * LPB>();
            else if (inflight == 1) wait_vm<NQ + LPB>();
            else wait_vm<NQ>();
        }
        // The frequency read is written out: the compiler would wait for every load in flight
        // before an LDS read it cannot tell apart from their destinations.
        float fr;
        {
            const uint32_t fa =
                (uint32_t)(uintptr_t)(__attribute__((address_space(3))) float*)&sfreq[w][lane];
            asm volatile("ds_read_b32 %0, %1\n\ts_waitcnt lgkmcnt(0)" : "=v"(fr) : "v"(fa) : "memory");
        }
        // Row rl of the workgroup's rows (uniform in the wave: its position is a scalar load).
        const auto* pos4 = (const __attribute__((address_space(4))) uint32_t*)p.positions;
#pragma unroll 1
        for (uint32_t rl = (uint32_t)w; rl < p.rb; rl += W) {
            const uint32_t r = r0 + rl;
            const float th = (float)pos4[r < p.rows ? r : 0u] * fr;
            float sn, cs;
            sincosf(th, &sn, &cs);
            rsc[rl * 64 + lane] = float2{sn, cs};
        }
    }
    // Q in (and the new rows), the blocks still in flight.
    if (inflight == 2)
        wait_vm<2 * LPB>();
    else if (inflight == 1)
        wait_vm<LPB>();
    else
        wait_vm<0>();
    if constexpr (FUSE) {
        // Everyone's table and new rows in (the barrier; no wait for the blocks in flight).
        __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
        barrier();
        // The new rows as the cache will hold them, K rotated by the table's row (pair (a, b):
        // neox (pp, pp + hr), else (2pp, 2pp + 1); y0 = x_a c - x_b s, y1 = x_a s + x_b c, as
        // k_rope_append), into nrow: thread tid takes row tid / 16, dims 8 (tid % 16) .. +7.
        if (has_new) {
            const uint32_t hr = p.rope_dim / 2, r = tid / 16, d0 = 8 * (tid % 16);
            if (r < p.rows) {
                const float* kx = raw + r * HD;
                const float* vx = raw + FUSE_ROWS * HD + r * HD;
                half8 kh, vh;
#pragma unroll
                for (int j = 0; j < 8; j++) {
                    const uint32_t d = d0 + j;
                    float y = kx[d];
                    if (d < p.rope_dim) {
                        const bool first = p.neox ? d < hr : (d & 1u) == 0u;
                        const uint32_t e = p.neox ? (first ? d + hr : d - hr) : (d ^ 1u);
                        const uint32_t pp = p.neox ? (first ? d : e) : d / 2;
                        const float2 t = rsc[(r - r0) * 64 + pp];
                        float y0, y1;
                        if (first)
                            rotate_sc(kx[d], kx[e], t.x, t.y, y0, y1);
                        else
                            rotate_sc(kx[e], kx[d], t.x, t.y, y0, y1);
                        y = first ? y0 : y1;
                    }
                    kh[j] = to_kv<f16>(y);
                    vh[j] = to_kv<f16>(vx[d]);
                }
                *(half8*)&nrow[0][r * HD + d0] = kh;
                *(half8*)&nrow[1][r * HD + d0] = vh;
            }
        }
        // nrow in before any block reads it, and every read of the staged rows in the third
        // stage done before its block's loads.
        __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
        barrier();
    }
    {
        const uint32_t qa = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) float*)&qlds[w][4 * lane];
        // FUSE: the sines and cosines of this lane's pairs (slot n's row) come in with Q, four
        // pairs a read: adjacent pairs 16 (k / 2) + 4 (lane / 16) + 0..3 (k = 0, 2, 4, 6), neox
        // pairs 32 (k / 2) + 8 (lane / 16) + 4 (k % 2) + 0..3 (k < 4; rope_dim 64 uses the
        // first two). The table's reads are written out too, and listed as operands of Q's
        // reads, whose wait covers them.
        f32x4 t4[FUSE ? 8 : 1];
        const uint32_t db = 8u * (uint32_t)(lane / 16);
        f32x4 qv[2 * NKC];
#define BCHIP_Q_READS(A)                                                              \
    "ds_read_b128 %0, %" #A "\n\tds_read_b128 %1, %" #A " offset:1024\n\t"            \
    "ds_read_b128 %2, %" #A " offset:2048\n\tds_read_b128 %3, %" #A " offset:3072\n\t" \
    "ds_read_b128 %4, %" #A " offset:4096\n\tds_read_b128 %5, %" #A " offset:5120\n\t" \
    "ds_read_b128 %6, %" #A " offset:6144\n\tds_read_b128 %7, %" #A " offset:7168\n\t"
        if constexpr (FUSE) {
            const uint32_t tb = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) float2*)&rsc[0] +
                                ((16u * w + n) % p.rb) * 512u;
            if (!p.neox)
                asm volatile(
                    "ds_read_b128 %0, %8\n\tds_read_b128 %1, %8 offset:16\n\t"
                    "ds_read_b128 %2, %8 offset:128\n\tds_read_b128 %3, %8 offset:144\n\t"
                    "ds_read_b128 %4, %8 offset:256\n\tds_read_b128 %5, %8 offset:272\n\t"
                    "ds_read_b128 %6, %8 offset:384\n\tds_read_b128 %7, %8 offset:400"
                    : "=&v"(t4[0]), "=&v"(t4[1]), "=&v"(t4[2]), "=&v"(t4[3]), "=&v"(t4[4]), "=&v"(t4[5]),
                      "=&v"(t4[6]), "=&v"(t4[7])
                    : "v"(tb + 4u * db)
                    : "memory");
            else
                asm volatile(
                    "ds_read_b128 %0, %8\n\tds_read_b128 %1, %8 offset:16\n\t"
                    "ds_read_b128 %2, %8 offset:32\n\tds_read_b128 %3, %8 offset:48\n\t"
                    "ds_read_b128 %4, %8 offset:256\n\tds_read_b128 %5, %8 offset:272\n\t"
                    "ds_read_b128 %6, %8 offset:288\n\tds_read_b128 %7, %8 offset:304"
                    : "=&v"(t4[0]), "=&v"(t4[1]), "=&v"(t4[2]), "=&v"(t4[3]), "=&v"(t4[4]), "=&v"(t4[5]),
                      "=&v"(t4[6]), "=&v"(t4[7])
                    : "v"(tb + 8u * db)
                    : "memory");
            asm volatile(BCHIP_Q_READS(16) "s_waitcnt lgkmcnt(0)"
                         : "=&v"(qv[0]), "=&v"(qv[1]), "=&v"(qv[2]), "=&v"(qv[3]), "=&v"(qv[4]), "=&v"(qv[5]),
                           "=&v"(qv[6]), "=&v"(qv[7]), "+v"(t4[0]), "+v"(t4[1]), "+v"(t4[2]), "+v"(t4[3]),
                           "+v"(t4[4]), "+v"(t4[5]), "+v"(t4[6]), "+v"(t4[7])
                         : "v"(qa)
                         : "memory");
        } else {
            asm volatile(BCHIP_Q_READS(8) "s_waitcnt lgkmcnt(0)"
                         : "=&v"(qv[0]), "=&v"(qv[1]), "=&v"(qv[2]), "=&v"(qv[3]), "=&v"(qv[4]), "=&v"(qv[5]),
                           "=&v"(qv[6]), "=&v"(qv[7])
                         : "v"(qa)
                         : "memory");
        }
#undef BCHIP_Q_READS
        static_assert(NKC == 4, "eight 1 KB rows of Q a wave");
        if constexpr (FUSE) {
            // Q rotated in registers as k_rope_append rotates it (the same expressions, so the
            // same bits): lane holds slot n's dims 32 (k / 2) + 8 (lane / 16) + 4 (k % 2) + j in
            // qv[k][j], so an adjacent pair is two elements of one register and a neox pair
            // (d, d + rope_dim / 2, rope_dim 64 or 128: the launch checks) the same element of
            // qv[k] and qv[k + rope_dim / 32]. Every rotation is computed, kept where the pair
            // is rotated (no branches on the lane's dims).
            if (!p.neox) {
#pragma unroll
                for (int k = 0; k < 2 * NKC; k++)
#pragma unroll
                    for (int j = 0; j < 4; j += 2) {
                        const uint32_t d = 32u * (k / 2) + db + 4u * (k % 2) + j;
                        const f32x4& t2 = t4[2 * (k / 2) + k % 2];  // pairs 2 (k % 2) + 0, 1
                        const float2 t = j == 0 ? float2{t2[0], t2[1]} : float2{t2[2], t2[3]};
                        float y0, y1;
                        rotate_sc(qv[k][j], qv[k][j + 1], t.x, t.y, y0, y1);
                        const bool rot = d < p.rope_dim;
                        qv[k][j] = rot ? y0 : qv[k][j];
                        qv[k][j + 1] = rot ? y1 : qv[k][j + 1];
                    }
            } else {
                auto rot = [&](auto KH) {
                    constexpr int kh = decltype(KH)::value;
#pragma unroll
                    for (int k = 0; k < kh; k++)
#pragma unroll
                        for (int j = 0; j < 4; j++) {
                            const f32x4& t2 = t4[2 * k + j / 2];
                            const float2 t = j % 2 == 0 ? float2{t2[0], t2[1]} : float2{t2[2], t2[3]};
                            float y0, y1;
                            rotate_sc(qv[k][j], qv[k + kh][j], t.x, t.y, y0, y1);
                            qv[k][j] = y0;
                            qv[k + kh][j] = y1;
                        }
                };
                if (p.rope_dim == 128)
                    rot(ic<4>{});
                else
                    rot(ic<2>{});
            }
            // The workgroup that writes the rotated Q back keeps it in its LDS rows until then
            // (written out, like the read).
            if (cs_idx == 0) {
                asm volatile(
                    "ds_write_b128 %0, %1\n\tds_write_b128 %0, %2 offset:1024\n\t"
                    "ds_write_b128 %0, %3 offset:2048\n\tds_write_b128 %0, %4 offset:3072\n\t"
                    "ds_write_b128 %0, %5 offset:4096\n\tds_write_b128 %0, %6 offset:5120\n\t"
                    "ds_write_b128 %0, %7 offset:6144\n\tds_write_b128 %0, %8 offset:7168"
                    :
                    : "v"(qa), "v"(qv[0]), "v"(qv[1]), "v"(qv[2]), "v"(qv[3]), "v"(qv[4]), "v"(qv[5]), "v"(qv[6]),
                      "v"(qv[7])
                    : "memory");
            }
        }
#pragma unroll
        for (int c = 0; c < NKC; c++) {
            const f32x4 a = qv[2 * c], b = qv[2 * c + 1];
            qb[c] = q_scaled(float4{a[0], a[1], a[2], a[3]}, float4{b[0], b[1], b[2], b[3]}, p.sc);
        }
    }

    // FUSE: this wave's rows of the block at key0 that are new (slot pos + r for row r of the
    // launch): K dims 8 (lane % 16 ^ swizzle) .. +7 and V's dims of the V load pattern, from
    // the staged rows (K rotated, both rounded to the cache type), into the stage (over what the
    // block's loads brought for those rows) and into the caches.
    auto new_rows = [&](uint32_t key0, f16* kl) {
        f16* vl = kl + BLK * HD;
#pragma unroll
        for (int i = 0; i < LPW; i++) {
            const uint32_t q = i * W + w, row = q * RPI + lane / PF_CPR, pch = lane % PF_CPR;
            const uint32_t key = key0 + row;
            if (key < p.pos || key >= kb1) continue;
            const uint32_t r = key - p.pos;
            const uint32_t dk = 8 * (pch ^ pf_kswz(row)), dv = 8 * (pch ^ pf_vswz(row));
            const half8 kh = *(const half8*)&nrow[0][r * HD + dk];
            const half8 vh = *(const half8*)&nrow[1][r * HD + dv];
            *(half8*)&kl[q * RPI * HD + 8 * lane] = kh;
            *(half8*)&vl[q * RPI * HD + 8 * lane] = vh;
            *(half8*)((f16*)p.kc + (size_t)key * kvd + (size_t)kvh * HD + dk) = kh;
            *(half8*)((f16*)p.vc + (size_t)key * kvd + (size_t)kvh * HD + dv) = vh;
        }
    };
    // One block in stage S: scores, mask, softmax, PV.
    auto iter = [&](uint32_t key0, auto S) -> bool {
        constexpr int s0 = decltype(S)::value;
        const uint32_t key1 = key0 + BLK;
        // This block in (own loads: wait, leaving the next block's in flight; everyone's:
        // the barrier), and every read of the stage that block b+2 refills (block b-1's) is
        // over.
        if (key1 < kb1)
            wait_vm<LPB>();
        else
            wait_vm<0>();
        if constexpr (FUSE) {
            // The launch's new rows in this block: each wave writes the rows its own loads
            // brought (they have landed), K rotated and V as the cache holds them, into the
            // stage and into the caches.
            if (key1 > p.pos) {
                new_rows(key0, ring(S));
                __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): the rows are in the stage
            }
        }
        barrier();
        load_block(key0 + (STAGES - 1) * BLK, ic<(s0 + STAGES - 1) % STAGES>{});
        // S^T = K . Q^T: four key tiles, hd chunks accumulated in order.
        const f16* kls = ring(S);
        f32x4 sc[4];
#pragma unroll
        for (int kt = 0; kt < 4; kt++) {
            sc[kt] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int c = 0; c < NKC; c++) sc[kt] = mfma16(*(const half8*)&kls[kbase[c] + kt * 16 * HD], qb[c], sc[kt]);
        }
        // Entries at or past a slot's list length are masked (a block every slot of the
        // tile sees whole skips the test).
        if (!__all(key0 + BLK <= len)) {
            keep_branch();
#pragma unroll
            for (int kt = 0; kt < 4; kt++)
#pragma unroll
                for (int i = 0; i < 4; i++)
                    if (key0 + 16 * kt + 4 * g + i >= len) sc[kt][i] = -INFINITY;
        }
        half8 pb[2];
        float corr;
        tile_softmax(cs, sc, pb, corr);
        rescale(cs.o, corr);
        // PV of the block.
        const f16* vls = ring(S) + BLK * HD;
#pragma unroll
        for (int kc = 0; kc < 2; kc++) {
            if constexpr (VT) {
#pragma unroll
                for (int dt = 0; dt < NDT; dt++)
                    cs.o[dt] = mfma16(*(const half8*)&vls[vbase[kc] + dt * 16 * BLK], pb[kc], cs.o[dt]);
            } else if constexpr (W == 4) {
                // Transposing reads (source lane j of its 16-lane group names row kbase + j/4,
                // dims 16dt + 4(j%4): chunk 2dt + (j%4)/2, half (j%4)%2), written out with one
                // wait per four dims tiles: the compiler's intrinsic would carry a wait for
                // every load in flight (it cannot tell these reads miss the stages still
                // filling), holding the block's PV until the block two ahead lands. This
                // stage's own loads landed before the block's barrier. Row r and r + 16 share
                // the swizzle, so a read's address is the lane's row base plus 16 dims' chunk
                // (dt ^ s) * 32 bytes, and the second half of the rows an immediate offset.
                static_assert(16 * HD * 2 == 4096, "lds_tr4x4's second rows sit 16 rows of hd 128 on");
                uint32_t rowb = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) const f16*)&vls[vrow + kc * 32 * HD];
                asm("" : "+v"(rowb));  // per block: not hoisted into registers for every stage
#pragma unroll
                for (int d0 = 0; d0 < NDT; d0 += 4) {
                    half4 lo[4], hi[4];
                    lds_tr4x4(lo, hi, rowb + 32u * ((uint32_t)(d0 + 0) ^ vsw), rowb + 32u * ((uint32_t)(d0 + 1) ^ vsw),
                              rowb + 32u * ((uint32_t)(d0 + 2) ^ vsw), rowb + 32u * ((uint32_t)(d0 + 3) ^ vsw));
#pragma unroll
                    for (int j = 0; j < 4; j++) {
                        const half8 a = half8{lo[j][0], lo[j][1], lo[j][2], lo[j][3], hi[j][0], hi[j][1], hi[j][2], hi[j][3]};
                        cs.o[d0 + j] = mfma16(a, pb[kc], cs.o[d0 + j]);
                    }
                }
            } else {
#pragma unroll
                for (int dt = 0; dt < NDT; dt++) {
                    // transposing read: source lane j of its 16-lane group names row
                    // kbase + j/4, dims 16dt + 4(j%4): chunk 2dt + (j%4)/2, half (j%4)%2
                    const uint32_t r = 32 * kc + 4 * g + (n >> 2), ch = 2 * dt + ((n & 3) >> 1), h = n & 1;
                    const half4 lo = lds_tr4(&vls[r * HD + 8 * (ch ^ pf_vswz(r)) + 4 * h]);
                    const uint32_t r2 = r + 16;
                    const half4 hi = lds_tr4(&vls[r2 * HD + 8 * (ch ^ pf_vswz(r2)) + 4 * h]);
                    const half8 a = half8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
                    cs.o[dt] = mfma16(a, pb[kc], cs.o[dt]);
                }
            }
        }
        return key1 < kb1;
    };
    // Chunk by chunk: three blocks, then (when the list goes on) the chunk's fold into R and
    // a fresh state.
    if (kb0 < kb1) {
        for (uint32_t key0 = kb0;; key0 += CHUNK_MULTI) {
            if (!iter(key0, ic<0>{})) break;
            if (!iter(key0 + BLK, ic<1>{})) break;
            if (!iter(key0 + 2 * BLK, ic<2>{})) break;
            fold(R, cs);
            state_clear(cs);
        }
    }
    if (p.split) {
        // The chunk's state: [unit][slot][HD] for attn_combine, [group][slot][chunk][HD] for
        // the group fold (a slot's chunks together).
        const uint32_t sl = 16 * w + n;
        const size_t at = p.gcnt ? ((size_t)grp * (16 * W) + sl) * p.nchunk + cs_idx
                                 : ((size_t)grp * p.nchunk + cs_idx) * (16 * W) + sl;
        // Streaming stores: the states are read once, by the fold (measured: the verify call at
        // 4096 slots 13.4 -> 13.0 us; a decode's chunk states, read by attn_row_fold, measured
        // slower so).
        float* po = p.part_o + at * HD;
#pragma unroll
        for (int dt = 0; dt < NDT; dt++) __builtin_nontemporal_store(cs.o[dt], (f32x4*)(po + 16 * dt + 4 * g));
        if (g == 0) *(float2*)(p.part_ml + at * 2) = float2{cs.m, cs.l};
        if (!p.gcnt) return;  // attn_combine folds the states
        // Group fold. Q's LDS rows are free for the flag word: each wave read its own rows
        // before its first block.
        GroupSync gsync{p.gcnt + (size_t)grp * GROUP_STRIDE, p.nchunk, p.gspins, p.gspread, 0u};
        uint32_t& flag = FUSE ? *(uint32_t*)&rsc[0] : *(uint32_t*)&qlds[0][0];
        uint32_t mode = group_arrive(gsync, p.gerr, flag);
        if (mode == GF_SPREAD) {
#pragma unroll
            for (int dt = 0; dt < NDT; dt++) store_wt4(po + 16 * dt + 4 * g, cs.o[dt]);
            if (g == 0) store_wt2(p.part_ml + at * 2, cs.m, cs.l);
            mode = group_second(gsync, p.gerr, flag);
        }
        if constexpr (FUSE) {
            // Every workgroup of the group has read its q: the first one leaves it rotated.
            if (cs_idx == 0 && valid && mode != GF_TIMEOUT) {
                float* dst = p.qw + ((size_t)orow * p.nh + ohead) * HD;
#pragma unroll
                for (int c = 0; c < NKC; c++)
#pragma unroll
                    for (int h = 0; h < 2; h++)
                        *(float4*)(dst + 32 * c + 8 * g + 4 * h) = *(const float4*)&qlds[w][(2 * c + h) * 256 + 4 * lane];
            }
        }
        // The ring's first stage is free: every wave is past its last block.
        group_fold_slots<16 * W>(p, grp, cs_idx, rbi, kvh, mode != GF_TIMEOUT, (float4*)ring0);
        if (mode != GF_TIMEOUT) group_leave(gsync);
        return;
    }
    fold(R, cs);
    if (!valid) return;
    float* o = p.out + ((size_t)orow * p.nh + ohead) * HD;
#pragma unroll
    for (int dt = 0; dt < NDT; dt++) {
        const uint32_t d = 16 * dt + 4 * g;
        *(float4*)(o + d) = float4{R.o[dt][0] / R.l, R.o[dt][1] / R.l, R.o[dt][2] / R.l, R.o[dt][3] / R.l};
    }
}

// The softmax of NT 16-slot tiles of a wave over one 64-entry block from relative scores
// y = s - m (the slot's running max already subtracted by the score MFMAs, whose
// accumulators start at -m), except in a list's first block (FIRST: y = s, and the block's
// max becomes m). The running max moves only when a block's relative max passes LAZY; P =
// 2^y rounded to f16; its block sum is a dot2 chain over the lane's pairs (key tiles in
// order), then the pairs across lanes l^16 and l^32 (block_step's order); O and l take the
// factor corr (1 where the max held). The tiles' steps interleave (each step of every tile
// before the next step), so that their dependency chains overlap in one wave.
template <int NDT, int NT, bool FIRST>
__device__ __forceinline__ void tiles_softmax_rel(State<NDT> (&s)[NT], f32x4 (&y)[NT][4], half8 (&pb)[NT][2]) {
    // The lane's max of each tile (a max is exact in any order).
    float lm[NT];
#pragma unroll
    for (int t = 0; t < NT; t++) {
        lm[t] = fmaxf(fmaxf(y[t][0][0], y[t][0][1]), fmaxf(y[t][0][2], y[t][0][3]));
#pragma unroll
        for (int kt = 1; kt < 4; kt++)
            lm[t] = fmaxf(lm[t], fmaxf(fmaxf(y[t][kt][0], y[t][kt][1]), fmaxf(y[t][kt][2], y[t][kt][3])));
    }
    float corr[NT];
    if constexpr (FIRST) {
#pragma unroll
        for (int t = 0; t < NT; t++) {
            const float my = xmax32(xmax16(lm[t]));
            const float ms = (my == -INFINITY) ? 0.0f : my;
            corr[t] = 1.0f;  // O and l are still zero
            s[t].m = my;
#pragma unroll
            for (int kt = 0; kt < 4; kt++)
#pragma unroll
                for (int i = 0; i < 4; i++) y[t][kt][i] = y[t][kt][i] - ms;
        }
    } else {
        // A slot's max moves only if its block max passes LAZY, and then some lane's own max
        // does: while no lane's does (most blocks of a long list), no slot's max moves, no
        // score shifts and O and l keep their scale, so the block skips the slots' maxima.
        bool maybe = false;
#pragma unroll
        for (int t = 0; t < NT; t++) {
            corr[t] = 1.0f;
            maybe = maybe || lm[t] > LAZY;
        }
        if (__any(maybe)) {
            keep_branch();
#pragma unroll
            for (int t = 0; t < NT; t++) {
                const float my = xmax32(xmax16(lm[t]));
                const bool up = my > LAZY;
                const float ms = up ? my : 0.0f;
                corr[t] = up ? exp2_hw(-my) : 1.0f;
                s[t].m = up ? s[t].m + my : s[t].m;
                // A slot whose max held subtracts 0 and multiplies by 1: exact.
#pragma unroll
                for (int kt = 0; kt < 4; kt++)
#pragma unroll
                    for (int i = 0; i < 4; i++) y[t][kt][i] = y[t][kt][i] - ms;
#pragma unroll
                for (int dt = 0; dt < NDT; dt++) s[t].o[dt] = s[t].o[dt] * corr[t];
            }
        }
    }
    uint32_t hp[NT][4][2];
    float ls[NT];
#pragma unroll
    for (int t = 0; t < NT; t++) ls[t] = 0.0f;
#pragma unroll
    for (int kt = 0; kt < 4; kt++)
#pragma unroll
        for (int j = 0; j < 2; j++)
#pragma unroll
            for (int t = 0; t < NT; t++) {
                const half2 h = half2{(f16)exp2_hw(y[t][kt][2 * j]), (f16)exp2_hw(y[t][kt][2 * j + 1])};
                ls[t] = pair_sum(h, ls[t]);
                hp[t][kt][j] = __builtin_bit_cast(uint32_t, h);
            }
    float ps[NT];
#pragma unroll
    for (int t = 0; t < NT; t++) ps[t] = xsum16(ls[t]);
#pragma unroll
    for (int t = 0; t < NT; t++) ps[t] = xsum32(ps[t]);
#pragma unroll
    for (int t = 0; t < NT; t++) s[t].l = s[t].l * corr[t] + ps[t];
#pragma unroll
    for (int t = 0; t < NT; t++)
#pragma unroll
        for (int kc = 0; kc < 2; kc++)
            pb[t][kc] = __builtin_bit_cast(half8, u32x4{hp[t][2 * kc][0], hp[t][2 * kc][1], hp[t][2 * kc + 1][0],
                                                        hp[t][2 * kc + 1][1]});
}

// Wide line passes (prefill) on f16 caches at hd 128: every row's list in one online softmax
// over 64-entry blocks from slot 0, one accumulator a slot (no chunk fold). Each wave takes
// two 16-slot tiles (32 query slots), so every K and V operand read from LDS feeds two
// MFMAs; a workgroup is four waves (128 slots: rows x the G heads of one KV head), and K and
// V^T (packed by vt_pack) blocks stream HBM -> LDS by direct-to-LDS loads through a ring of
// two stages (32 KB each), one block ahead. At 64 KB of LDS and at most 256 registers a lane,
// two workgroups share a CU, one wave of each on every SIMD; the two are not synchronised
// with each other, so one's softmax runs beside the other's MFMAs.
// The arithmetic per slot is block_step's (scores by 16x16x32 f16 MFMAs in log2 units, the
// lazy running max, P rounded to f16 once, PV into the same accumulator; the score MFMAs'
// accumulators start at -m, so the running max rides in them); a row's bits depend only on
// its q and its list, never on the rows beside it.
// The loop is mostly one wave's chain of dependent steps (scores, softmax, PV), which the
// other wave on the SIMD hides only in part, so the schedule shortens that chain:
//  - the K operands are read from LDS two hd chunks ahead of the MFMAs that take them (eight
//    operands in flight), and the first V^T operands during the last score MFMAs;
//  - the two tiles' softmax steps interleave (tiles_softmax_rel), one branch for both;
//  - the list's first block is a copy of its own (no test of it in the loop).
template <int NT>
__global__ __launch_bounds__(256, 2) void attn_line(const SharedParams p) {
    constexpr int HD = 128;
    constexpr int NKC = HD / 32, NDT = HD / 16, W = 4;
    constexpr int RPI = 64 / PF_CPR;            // cache rows per load instruction
    constexpr int LPW = BLK / RPI / W;          // load instructions per wave per block (K or V)
    constexpr int SZ = 2 * BLK * HD;            // f16 per stage: K rows, then V (or V^T)
    static_assert(LPW * RPI * W == BLK, "a block's rows divide over the waves");
    static_assert(NKC == 4, "the score phase below reads K two hd chunks ahead of four");
    __shared__ __attribute__((aligned(16))) f16 ring0[SZ];
    __shared__ __attribute__((aligned(16))) f16 ring1[SZ];

    const int tid = threadIdx.x, lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int g = lane >> 4, n = lane & 15;
    const uint32_t kvh = blockIdx.x % p.nkv;
    const uint32_t rbi = p.nrb - 1u - blockIdx.x / p.nkv;  // heavy row blocks first
    const uint32_t r0 = rbi * p.rb;
    const uint32_t rlast = min(r0 + p.rb, p.rows) - 1u;
    const uint32_t maxlen = p.pos + rlast + 1u;
    const uint32_t kvd = p.nkv * HD;

    half8 qb[NT][NKC];
    float4 qraw[NT][NKC][2];
    uint32_t len[NT], orow[NT], ohead[NT];
    bool valid[NT];
#pragma unroll
    for (int t = 0; t < NT; t++) {
        const uint32_t sl = 16 * NT * w + 16 * t + n;
        const uint32_t gh = sl / p.rb, rl = sl % p.rb, r = r0 + rl;
        valid[t] = gh < p.G && r < p.rows;
        len[t] = valid[t] ? p.pos + r + 1u : maxlen;  // a slot with no row: zero q, no mask
        orow[t] = r;
        ohead[t] = kvh * p.G + gh;
        const float* qrow = valid[t] ? p.q + ((size_t)r * p.nh + ohead[t]) * HD : (const float*)p.zero;
#pragma unroll
        for (int c = 0; c < NKC; c++) {
            const float* src = valid[t] ? qrow + 32 * c + 8 * g : qrow;
            qraw[t][c][0] = *(const float4*)src;
            qraw[t][c][1] = *(const float4*)(src + 4);
        }
    }

    const f16* zp = (const f16*)p.zero;
    const f16* kcb = (const f16*)p.kc + (size_t)kvh * HD;
    const f16* vcb = (const f16*)p.vt + (size_t)kvh * HD * p.vt_npad;
    // Byte offsets of this wave's load instructions from a block's K rows and V^T columns,
    // fixed for the loop (32-bit, beside a scalar block base: no 64-bit address arithmetic
    // a block): K row 4q + l/16 (q = i*W + w), 16-byte chunk l%16 swizzled by the row; V^T
    // dim row 8q + l/8, chunk l%8 swizzled by the dim row.
    // Byte offsets of this wave's load instructions from a block's first K row and V^T column,
    // fixed for the loop: K row 4q + l/16 (q = i*W + w), 16-byte chunk l%16 swizzled by the
    // row; V^T dim row 8q + l/8, chunk l%8 swizzled by the dim row.
    uint32_t krow[LPW], koff[LPW], voff[LPW];
#pragma unroll
    for (int i = 0; i < LPW; i++) {
        const uint32_t q = i * W + w, row = q * RPI + lane / PF_CPR, pch = lane % PF_CPR;
        krow[i] = row;
        koff[i] = 2 * (row * kvd + 8 * (pch ^ pf_kswz(row)));
        const uint32_t d = q * 8 + lane / 8;
        voff[i] = 2 * (d * p.vt_npad + 8 * ((lane % 8) ^ (d % 8)));
    }
    typedef __attribute__((address_space(3))) void lds_t;
    auto load_block = [&](uint32_t key0, f16* kl) {
        f16* vl = kl + BLK * HD;
        const char* kb = (const char*)(kcb + (size_t)key0 * kvd);
        const char* vb = (const char*)(vcb + key0);
        if (key0 + BLK <= maxlen) {
            // A whole block: buffer loads from the block's bases (scalar), so the per-lane
            // offsets stay 32-bit registers fixed for the loop.
            const __amdgpu_buffer_rsrc_t kr = __builtin_amdgcn_make_buffer_rsrc((void*)kb, (short)0, 0x7fffffff, 0x00020000);
            const __amdgpu_buffer_rsrc_t vr = __builtin_amdgcn_make_buffer_rsrc((void*)vb, (short)0, 0x7fffffff, 0x00020000);
#pragma unroll
            for (int i = 0; i < LPW; i++) {
                const uint32_t q = i * W + w;
                __builtin_amdgcn_raw_ptr_buffer_load_lds(kr, (lds_t*)&kl[q * RPI * HD], 16, koff[i], 0, 0, 0);
                __builtin_amdgcn_raw_ptr_buffer_load_lds(vr, (lds_t*)&vl[q * 8 * BLK], 16, voff[i], 0, 0, 0);
            }
        } else {
            // The list's last block: K rows past it read the zero page (the packed V^T holds
            // zeros there already).
#pragma unroll
            for (int i = 0; i < LPW; i++) {
                const uint32_t q = i * W + w;
                const bool ok = key0 + krow[i] < maxlen;
                const void* ks = ok ? (const void*)(kb + koff[i]) : (const void*)(zp + 8 * (lane % PF_CPR));
                __builtin_amdgcn_global_load_lds(ks, (lds_t*)&kl[q * RPI * HD], 16, 0, 0);
                __builtin_amdgcn_global_load_lds((const void*)(vb + voff[i]), (lds_t*)&vl[q * 8 * BLK], 16, 0, 0);
            }
        }
    };
    uint32_t kbase[NKC], vbase[2];
#pragma unroll
    for (int c = 0; c < NKC; c++) kbase[c] = n * HD + 8 * ((4 * c + g) ^ n);
#pragma unroll
    for (int kc = 0; kc < 2; kc++) vbase[kc] = n * BLK + 8 * ((4 * kc + g) ^ (n % 8));
    auto barrier = [&]() {
        __builtin_amdgcn_sched_barrier(0);
        __builtin_amdgcn_s_barrier();
        __builtin_amdgcn_sched_barrier(0);
    };

    State<NDT> st[NT];
#pragma unroll
    for (int t = 0; t < NT; t++) state_clear(st[t]);
    load_block(0, ring0);
#pragma unroll
    for (int t = 0; t < NT; t++)
#pragma unroll
        for (int c = 0; c < NKC; c++) qb[t][c] = q_scaled(qraw[t][c][0], qraw[t][c][1], p.sc);

    auto iter = [&](uint32_t key0, const f16* kls, f16* nxt, auto FIRST) {
        constexpr bool first = decltype(FIRST)::value;
        // This block in (own loads: the wait; everyone's: the barrier, after which no wave
        // reads the other stage any more), the next block's loads out into it.
        wait_vm<0>();
        barrier();
        if (key0 + BLK < maxlen) load_block(key0 + BLK, nxt);
        auto kop = [&](int kt, int c) { return *(const half8*)&kls[kbase[c] + kt * 16 * HD]; };
        const f16* vls = kls + BLK * HD;
        auto vop = [&](int dt, int kc) { return *(const half8*)&vls[vbase[kc] + dt * 16 * BLK]; };
        f32x4 sc[NT][4];
#pragma unroll
        for (int t = 0; t < NT; t++) {
            const float nm = first ? 0.0f : -st[t].m;
#pragma unroll
            for (int kt = 0; kt < 4; kt++) sc[t][kt] = f32x4{nm, nm, nm, nm};
        }
        // Scores, hd chunks in order; chunk c's K operands were read two chunks earlier.
        half8 ka[2][4];
#pragma unroll
        for (int kt = 0; kt < 4; kt++) ka[0][kt] = kop(kt, 0);
#pragma unroll
        for (int kt = 0; kt < 4; kt++) ka[1][kt] = kop(kt, 1);
        half8 va[NDT];
#pragma unroll
        for (int c = 0; c < NKC; c++) {
#pragma unroll
            for (int kt = 0; kt < 4; kt++)
#pragma unroll
                for (int t = 0; t < NT; t++) sc[t][kt] = mfma16(ka[c & 1][kt], qb[t][c], sc[t][kt]);
            if (c + 2 < NKC) {
#pragma unroll
                for (int kt = 0; kt < 4; kt++) ka[c & 1][kt] = kop(kt, c + 2);
            }
            if (c == NKC - 2) {
#pragma unroll
                for (int dt = 0; dt < NDT; dt++) va[dt] = vop(dt, 0);
            }
        }
        // LDS reads and MFMAs in this order: K chunks 0 and 1; MFMAs of chunk 0; K chunk 2;
        // MFMAs of chunk 1; K chunk 3; MFMAs of chunk 2; V^T of the first key half; MFMAs of
        // chunk 3.
        constexpr int MPC = 4 * NT;  // MFMAs a chunk
        __builtin_amdgcn_sched_group_barrier(0x100, 8, 0);
        __builtin_amdgcn_sched_group_barrier(0x008, MPC, 0);
        __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);
        __builtin_amdgcn_sched_group_barrier(0x008, MPC, 0);
        __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);
        __builtin_amdgcn_sched_group_barrier(0x008, MPC, 0);
        __builtin_amdgcn_sched_group_barrier(0x100, NDT, 0);
        __builtin_amdgcn_sched_group_barrier(0x008, MPC, 0);
        // Entries at or past a slot's list length are masked: one test for all tiles (a tile
        // every slot of which sees the whole block keeps its scores).
        bool edge = false;
#pragma unroll
        for (int t = 0; t < NT; t++) edge = edge || key0 + BLK > len[t];
        if (__any(edge)) {
            keep_branch();
#pragma unroll
            for (int t = 0; t < NT; t++)
#pragma unroll
                for (int kt = 0; kt < 4; kt++)
#pragma unroll
                    for (int i = 0; i < 4; i++)
                        if (key0 + 16 * kt + 4 * g + i >= len[t]) sc[t][kt][i] = -INFINITY;
        }
        half8 pb[NT][2];
        tiles_softmax_rel<NDT, NT, first>(st, sc, pb);
        half8 vb[NDT];
#pragma unroll
        for (int dt = 0; dt < NDT; dt++) vb[dt] = vop(dt, 1);
#pragma unroll
        for (int dt = 0; dt < NDT; dt++)
#pragma unroll
            for (int t = 0; t < NT; t++) st[t].o[dt] = mfma16(va[dt], pb[t][0], st[t].o[dt]);
#pragma unroll
        for (int dt = 0; dt < NDT; dt++)
#pragma unroll
            for (int t = 0; t < NT; t++) st[t].o[dt] = mfma16(vb[dt], pb[t][1], st[t].o[dt]);
    };
    iter(0u, ring0, ring1, std::true_type{});
    if (BLK < maxlen) {
        for (uint32_t key0 = BLK;; key0 += 2 * BLK) {
            iter(key0, ring1, ring0, std::false_type{});
            if (key0 + BLK >= maxlen) break;
            iter(key0 + BLK, ring0, ring1, std::false_type{});
            if (key0 + 2 * BLK >= maxlen) break;
        }
    }
#pragma unroll
    for (int t = 0; t < NT; t++) {
        if (!valid[t]) continue;
        float* o = p.out + ((size_t)orow[t] * p.nh + ohead[t]) * HD;
#pragma unroll
        for (int dt = 0; dt < NDT; dt++) {
            const uint32_t d = 16 * dt + 4 * g;
            *(float4*)(o + d) = float4{st[t].o[dt][0] / st[t].l, st[t].o[dt][1] / st[t].l, st[t].o[dt][2] / st[t].l,
                                       st[t].o[dt][3] / st[t].l};
        }
    }
}

// ---------------------------------------------------------------------------------------
// Launch plans.

static uint32_t ceil_div(uint64_t a, uint64_t b) { return (uint32_t)((a + b - 1) / b); }

template <int HD>
static hipError_t launch_combine_t(CombineParams& cp, uint32_t groups, hipStream_t s) {
    cp.ngroups = groups;
    // Lists of more than CMB_RUN chunks: the long fold, a workgroup per output slot.
    uint32_t most = cp.shared ? cp.nchunk : 0u;
    if (!cp.shared)
        for (uint32_t i = 0; i < cp.nitems; i++) most = std::max(most, cp.items[i].nchunk);
    if (cp.long_fold && most > (uint32_t)CMB_RUN) {
        hipLaunchKernelGGL((attn_combine_long<HD>), dim3((uint64_t)groups * cp.slots_out), dim3(CMBL_THREADS), 0, s, cp);
        return hipGetLastError();
    }
    const uint64_t threads = (uint64_t)groups * cp.slots_out * (cp.hd / 4);
    const dim3 grid(ceil_div(threads, CMB_THREADS)), block(CMB_THREADS);
    const uint32_t nc = cp.shared ? cp.nchunk : (uint32_t)CMB_RUN;
    if (nc <= 8)
        hipLaunchKernelGGL((attn_combine<HD, 8>), grid, block, 0, s, cp);
    else if (nc <= 16)
        hipLaunchKernelGGL((attn_combine<HD, 16>), grid, block, 0, s, cp);
    else if (nc <= 24)
        hipLaunchKernelGGL((attn_combine<HD, 24>), grid, block, 0, s, cp);
    else
        hipLaunchKernelGGL((attn_combine<HD, CMB_RUN>), grid, block, 0, s, cp);
    return hipGetLastError();
}

template <int HD, typename KVT, int W, int NT>
static hipError_t launch_shared_t(const SharedParams& sp, uint32_t blocks, const AttnCall& a, hipStream_t s) {
    hipExtLaunchKernelGGL((attn_shared<HD, KVT, W, NT>), dim3(blocks), dim3(64 * W), 0, s, a.ev_before, a.ev_after, 0, sp);
    return hipGetLastError();
}

static int pad_hd(uint32_t hd) {
    if (hd <= 32) return 32;
    if (hd <= 64) return 64;
    if (hd <= 128) return 128;
    return 256;
}

#define BCHIP_DISPATCH_HD(hdp, CALL)                       \
    switch (hdp) {                                         \
        case 32: { constexpr int HD = 32; CALL; } break;   \
        case 64: { constexpr int HD = 64; CALL; } break;   \
        case 128: { constexpr int HD = 128; CALL; } break; \
        default: { constexpr int HD = 256; CALL; } break;  \
    }

template <int HD>
static hipError_t launch_combine_t(CombineParams& cp, uint32_t groups, hipStream_t s);

hipError_t combine_launch(CombineParams& cp, uint32_t groups, uint32_t hd, hipStream_t s) {
    hipError_t e;
    BCHIP_DISPATCH_HD(pad_hd(hd), e = (launch_combine_t<HD>(cp, groups, s)));
    return e;
}

template <int HD, typename KVT>
static hipError_t launch_decode_t(DirectParams& dp, CombineParams& cp, const AttnCall& a, hipStream_t s) {
    // Tree rows only: lines of any length go to the shared kernels, one-row lists to the
    // one-row kernel.
    hipExtLaunchKernelGGL((attn_decode<HD, KVT>), dim3(dp.nunits), dim3(256), 0, s, a.ev_before, a.ev_after, 0, dp);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    return launch_combine_t<HD>(cp, dp.nitems * dp.nkv, s);
}

template <int HD, typename KVT>
static hipError_t launch_row_t(const DirectParams& dp, bool fold, const AttnCall& a, hipStream_t s) {
    const dim3 grid(ceil_div(dp.nunits, 4)), block(256);
    if (dp.fuse && dp.runs)
        hipExtLaunchKernelGGL((attn_decode_row<HD, KVT, true, true>), grid, block, 0, s, a.ev_before, a.ev_after, 0, dp);
    else if (dp.fuse)
        hipExtLaunchKernelGGL((attn_decode_row<HD, KVT, true, false>), grid, block, 0, s, a.ev_before, a.ev_after, 0, dp);
    else if (dp.runs)
        hipExtLaunchKernelGGL((attn_decode_row<HD, KVT, false, true>), grid, block, 0, s, a.ev_before, a.ev_after, 0, dp);
    else
        hipExtLaunchKernelGGL((attn_decode_row<HD, KVT, false, false>), grid, block, 0, s, a.ev_before, a.ev_after, 0, dp);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || !fold) return e;
    const uint32_t slices = (HD + ROW_FOLD_DIMS - 1) / ROW_FOLD_DIMS;
    hipLaunchKernelGGL((attn_row_fold<HD>), dim3(dp.nitems * dp.nkv * dp.G * slices), dim3(ROW_FOLD_THREADS), 0, s, dp);
    return hipGetLastError();
}

static DirectParams direct_params(const AttnCall& a, const Workspace& ws, uint32_t nitems) {
    DirectParams dp{};
    dp.zero = ws.zero;
    dp.q = a.q;
    dp.kc = a.kc;
    dp.vc = a.vc;
    dp.out = a.out;
    dp.masks = a.masks;
    dp.slot_limit = a.slot_limit;
    dp.nh = a.nh;
    dp.nkv = a.nkv;
    dp.hd = a.hd;
    dp.G = a.nh / a.nkv;
    dp.base = a.pos;
    dp.tree = a.tree;
    dp.sc = a.scale * LOG2E;
    dp.nitems = nitems;
    return dp;
}

// Chunk of a one-row list with nkv KV heads (each (chunk, KV head) is one wave's unit):
// a multiple of RB (at least two blocks) that cuts the list into at most ROW_UNITS / nkv
// chunks, and at most ROW_MAX_CHUNKS. A long step then has about ROW_UNITS waves, four per
// CU, all issuing their loads from the start. Measured, decode kernel at 32768 slots x 8 KV
// heads: ROW_UNITS 768: 26.9 us, 896: 26.5, 1024 (912 units of 288 entries): 24.9, 1536:
// 30.2, 2048: 26.4; 1024 units of 257 entries (not a multiple of RB; 256 workgroups): 28.0.
// It depends only on the list's own length and nkv, so a sequence gets the same bits in any
// ragged batch as alone.
constexpr uint64_t ROW_UNITS = 1024;

uint32_t row_chunk(uint64_t len, uint32_t nkv) {
    uint64_t most = std::max<uint64_t>(1, ROW_UNITS / std::max<uint32_t>(nkv, 1));
    most = std::min<uint64_t>(most, ROW_MAX_CHUNKS);
    uint64_t chunk = (len + most - 1) / most;
    chunk = (chunk + RB - 1) / RB * RB;
    return (uint32_t)std::max<uint64_t>(chunk, 2 * RB);
}

size_t row_state_slots(uint64_t len, uint32_t nkv) {
    const uint64_t chunk = row_chunk(len, nkv);
    return (size_t)nkv * ((len + chunk - 1) / chunk) * 16;
}

bool row_fusable(uint32_t nh, uint32_t nkv, uint32_t hd, uint32_t rope_dim, uint32_t neox) {
    // The shapes the fused kernel is built and tested for: whole 32-dim operand groups, neox
    // halves of whole groups, and at most ROW_FUSE_MAXG query heads per KV head (each lane
    // holds its pairs of every head of the group in registers); others run as the two calls.
    return nkv > 0 && nh % nkv == 0 && nh / nkv <= ROW_FUSE_MAXG && hd % 32 == 0 && hd <= MAX_HD &&
           rope_dim % 2 == 0 && rope_dim <= hd && (!neox || (rope_dim / 2) % 32 == 0);
}

static hipError_t row_launch(const AttnCall& a, const Item* items, uint32_t nitems, const RopeArgs* rope,
                             Workspace& ws, hipStream_t s);

hipError_t row_attention(const AttnCall& a, const Item* items, uint32_t nitems, Workspace& ws, hipStream_t s) {
    return row_launch(a, items, nitems, nullptr, ws, s);
}

hipError_t row_attention_fused(const AttnCall& a, const RopeArgs& r, Workspace& ws, hipStream_t s) {
    if (!row_fusable(a.nh, a.nkv, a.hd, r.rope_dim, r.neox)) return hipErrorInvalidValue;
    Item item{};
    item.row = 0;
    item.nrows = 1;
    item.len = a.pos + 1;
    return row_launch(a, &item, 1, &r, ws, s);
}

hipError_t row_attention_fused_items(const AttnCall& a, const RopeArgs& r, const Item* items, uint32_t nitems,
                                     Workspace& ws, hipStream_t s) {
    if (!row_fusable(a.nh, a.nkv, a.hd, r.rope_dim, r.neox)) return hipErrorInvalidValue;
    return row_launch(a, items, nitems, &r, ws, s);
}

static hipError_t row_launch(const AttnCall& a, const Item* items, uint32_t nitems, const RopeArgs* rope,
                             Workspace& ws, hipStream_t s) {
    if (nitems == 0 || nitems > MAX_ITEMS) return hipErrorInvalidValue;
    DirectParams dp = direct_params(a, ws, nitems);
    dp.tree = 0;
    if (rope) {
        dp.fuse = 1;
        dp.qw = rope->q;
        dp.knew = rope->k;
        dp.vnew = rope->v;
        dp.inv_freq = rope->inv_freq;
        dp.positions = rope->positions;
        dp.rope_dim = rope->rope_dim;
        dp.neox = rope->neox;
    }
    uint64_t units = 0;
    bool fold = false;
    for (uint32_t i = 0; i < nitems; i++) {
        Item& I = dp.items[i];
        I = items[i];
        if (I.len == 0) return hipErrorInvalidValue;
        I.nrows = 1;
        I.chunk = row_chunk(I.len, a.nkv);
        I.nchunk = ceil_div(I.len, I.chunk);
        units += (uint64_t)a.nkv * I.nchunk;
        fold = fold || I.nchunk > 1;
    }
    // A unit a chunk, or a unit a run of ROW_RUN chunks for a launch of 4 ROW_UNITS chunk
    // units or more (a ragged batch of long lists).
    dp.runs = ws.row_runs == 2 || (ws.row_runs == 1 && units >= 4 * ROW_UNITS);
    // The items of the longest chunks first, so that the launch's last workgroups are its
    // shortest (an item's place in the launch changes none of its arithmetic).
    std::stable_sort(dp.items, dp.items + nitems, [](const Item& x, const Item& y) { return x.chunk > y.chunk; });
    units = 0;
    for (uint32_t i = 0; i < nitems; i++) {
        Item& I = dp.items[i];
        I.unit0 = (uint32_t)units;
        units += (uint64_t)a.nkv * (dp.runs ? ceil_div(I.nchunk, ROW_RUN) : I.nchunk);
    }
    if (units > 0x7fffffffull) return hipErrorInvalidValue;
    dp.nunits = (uint32_t)units;
    const int hdp = pad_hd(a.hd);
    hipError_t e = ws.reserve((size_t)units * 16, (size_t)hdp);
    if (e == hipSuccess && rope) e = ws.reserve_qrot((size_t)nitems * a.nh * a.hd);
    if (e != hipSuccess) return e;
    dp.part_o = ws.o;
    dp.part_ml = ws.ml;
    dp.qrot = ws.qrot;
    // f16 caches only: f32 caches take the f32 path (attention_f32.hip).
    if (a.kv_type != 1) return hipErrorInvalidValue;
    BCHIP_DISPATCH_HD(hdp, e = (launch_row_t<HD, f16>(dp, fold, a, s)));
    return e;
}

// Multi-row passes of decode-kernel units (tree rows, a few line rows): chunk states folded
// left to right by attn_combine, as every multi-row line is, so that a tree row matches its
// line bit for bit.
hipError_t direct_attention(const AttnCall& a, const Item* items, uint32_t nitems, Workspace& ws, hipStream_t s) {
    if (nitems == 0 || nitems > MAX_ITEMS) return hipErrorInvalidValue;
    DirectParams dp = direct_params(a, ws, nitems);
    uint32_t units = 0;
    const int hdp = pad_hd(a.hd);
    for (uint32_t i = 0; i < nitems; i++) {
        Item& I = dp.items[i];
        I = items[i];
        I.unit0 = units;
        units += a.nkv * I.nchunk;
    }
    dp.nunits = units;
    hipError_t e = ws.reserve((size_t)units * 16, (size_t)hdp);
    if (e != hipSuccess) return e;
    dp.part_o = ws.o;
    dp.part_ml = ws.ml;
    CombineParams cp{};
    cp.long_fold = ws.combine_long;
    cp.zero = ws.zero;
    cp.out = a.out;
    cp.part_o = ws.o;
    cp.part_ml = ws.ml;
    cp.nh = a.nh;
    cp.nkv = a.nkv;
    cp.hd = a.hd;
    cp.G = dp.G;
    cp.slots = 16;
    cp.slots_out = 16;
    cp.shared = 0;
    cp.nitems = nitems;
    for (uint32_t i = 0; i < nitems; i++) cp.items[i] = dp.items[i];
    if (a.kv_type != 1) return hipErrorInvalidValue;
    BCHIP_DISPATCH_HD(hdp, e = (launch_decode_t<HD, f16>(dp, cp, a, s)));
    return e;
}

static hipError_t shared_plan(const AttnCall& a, Workspace& ws, hipStream_t s, const RopeArgs* rope);

hipError_t shared_attention(const AttnCall& a, Workspace& ws, hipStream_t s) { return shared_plan(a, ws, s, nullptr); }

hipError_t shared_attention_fused(const AttnCall& a, const RopeArgs& r, Workspace& ws, hipStream_t s) {
    return shared_plan(a, ws, s, &r);
}

static hipError_t shared_plan(const AttnCall& a, Workspace& ws, hipStream_t s, const RopeArgs* rope) {
    SharedParams sp{};
    sp.zero = ws.zero;
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
        // (GFOLD_MAX_CHUNKS states to spare past the last: the group fold's loads run past a
        // slot's last chunk.)
        hipError_t e = ws.reserve((size_t)groups * sp.nchunk * SL + GFOLD_MAX_CHUNKS, (size_t)hdp);
        if (e != hipSuccess) return e;
        sp.part_o = ws.o;
        sp.part_ml = ws.ml;
    }
    const uint32_t blocks = groups * (sp.split ? sp.nchunk : 1u);
    // The group fold (see group_arrive_wait) for split passes of the f16 hd-128 kernels whose
    // workgroups can all be resident at once: one a CU (their LDS takes most of one), at most
    // the device's CU count.
    const bool gfold = sp.split && a.kv_type == 1 && a.hd == 128 && ws.group_fold && ws.gcnt && blocks <= ws.cus &&
                       sp.nchunk <= GFOLD_MAX_CHUNKS && groups <= GROUP_COUNTERS;
    if (gfold) {
        sp.gcnt = ws.gcnt;
        sp.gerr = ws.gerr;
        sp.xmap = groups % 8 == 0;  // each XCD's share of blocks then holds whole groups
        sp.gspread = ws.group_spread;
        sp.gspins = ws.group_spins;
    }
    hipError_t e;
    if (rope) {
        // The fused form: one row block (every row's q rotated by the workgroups that read it),
        // the split pass's group fold (the rotated q is written once every workgroup of a group
        // has read it), the table of one row block's rotations, neox pairs a multiple of 32
        // dims apart (q is rotated in the registers it is read into).
        if (!(gfold && !wide && a.kv_type == 1 && a.hd == 128 && sp.nrb == 1 && sp.rb <= FUSE_ROWS &&
              rope->rope_dim <= a.hd && (!rope->neox || rope->rope_dim == 64 || rope->rope_dim == 128)))
            return hipErrorNotSupported;
        sp.knew = rope->k;
        sp.vnew = rope->v;
        sp.inv_freq = rope->inv_freq;
        sp.positions = rope->positions;
        sp.rope_dim = rope->rope_dim;
        sp.neox = rope->neox;
        sp.qw = rope->q;
        hipExtLaunchKernelGGL((attn_prefill<4, false, true>), dim3(blocks), dim3(256), 0, s, a.ev_before, a.ev_after, 0, sp);
        return hipGetLastError();
    }
    if (a.kv_type == 1 && a.hd == 128) {
        if (wide && !sp.split) {
            // The wide kernel, two 16-slot tiles a wave, four waves: 128 slots a workgroup as
            // sp.rb is sized, over V transposed once (a pass over V, vt_pack), so that its
            // operands are plain LDS reads: from 2048 rows the pass pays for itself (2048 rows
            // of 32/8 heads: 55.8 us of the wide kernel against 61.7 with transposing reads).
            SharedParams lp = sp;
            const uint32_t nb = ceil_div(maxlen, 64);
            lp.vt_npad = nb * 64;
            e = ws.reserve_vt((size_t)a.nkv * 128 * lp.vt_npad * 2);
            if (e != hipSuccess) return e;
            lp.vt = ws.vt;
            hipLaunchKernelGGL(vt_pack, dim3(nb, a.nkv), dim3(256), 0, s, (const f16*)a.vc,
                               (f16*)ws.vt, a.nkv * 128u, (uint32_t)maxlen, lp.vt_npad);
            e = hipGetLastError();
            if (e != hipSuccess) return e;
            hipExtLaunchKernelGGL((attn_line<2>), dim3(blocks), dim3(256), 0, s, a.ev_before, a.ev_after, 0, lp);
        } else if (wide) {
            hipExtLaunchKernelGGL((attn_prefill<8, false, false>), dim3(blocks), dim3(512), 0, s, a.ev_before, a.ev_after, 0, sp);
        } else {
            hipExtLaunchKernelGGL((attn_prefill<4, false, false>), dim3(blocks), dim3(256), 0, s, a.ev_before, a.ev_after, 0, sp);
        }
        e = hipGetLastError();
    } else if (a.kv_type == 1) {
        if (wide) {
            BCHIP_DISPATCH_HD(hdp, e = (launch_shared_t<HD, f16, 4, (HD <= 128 ? 2 : 1)>(sp, blocks, a, s)));
        } else {
            BCHIP_DISPATCH_HD(hdp, e = (launch_shared_t<HD, f16, 4, 1>(sp, blocks, a, s)));
        }
    } else {
        return hipErrorInvalidValue;  // f32 caches take the f32 path (attention_f32.hip)
    }
    if (e != hipSuccess || !sp.split || gfold) return e;
    CombineParams cp{};
    cp.long_fold = ws.combine_long;
    cp.zero = ws.zero;
    cp.out = a.out;
    cp.part_o = ws.o;
    cp.part_ml = ws.ml;
    cp.nh = a.nh;
    cp.nkv = a.nkv;
    cp.hd = a.hd;
    cp.G = sp.G;
    cp.slots = SL;
    cp.slots_out = SL;
    cp.shared = 1;
    cp.rows = a.rows;
    cp.rb = sp.rb;
    cp.nrb = sp.nrb;
    cp.nchunk = sp.nchunk;
    BCHIP_DISPATCH_HD(hdp, e = (launch_combine_t<HD>(cp, groups, s)));
    return e;
}

}  // namespace bchip
