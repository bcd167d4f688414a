// Attention over an f32 cache in f32 arithmetic: the path for callers that keep bc-infer's
// own f32 cache (crates/bc-infer/src/gpu/mod.rs:409-421) and want its results to f32
// rounding, as the reference's end-to-end tests demand (model.rs:531, 548, 642: 1e-4).
//
// The reference per (row, head) (model.rs:448-481): scores dot(q, k) * scale with
// quant::dot's eight lane sums (quant.rs:617-631), one softmax over the whole list, then
// o += (p / sum) v in slot order. Here the scores are the same dot (eight lanes summed in
// the same order, no fused multiply-add), times scale * log2(e); the softmax is online, over
// blocks of F32_BLK list entries in exp2 units: per block and slot, the block's max, the new
// running max, P = 2^(s - max), the block's sum of P and of P v (each in entry order), and
// the running state scaled by 2^(old max - new max). Lists go in chunks of CHUNK_MULTI
// entries, each an online softmax from a fresh state, folded left to right (merge_coef, the
// fold every other kernel and attn_combine use). A row's bits therefore depend only on its q
// and its list: the same in any batch, as a tree node or a line token, split over
// workgroups or not, and a one-row pass gives the bits of the same row in a batch.
//
// A workgroup holds F32_SLOTS query slots of one KV head (rows x heads of the group; one row
// for a tree), stages q and each block's K and V in LDS once for all of them, and walks its
// list's chunks (all of them, folding as it goes, or one, its state then folded by
// attn_combine when there are few workgroups). Bound: latency and LDS for the shapes this
// path serves (the reference's tests, config 1's decode); f16 caches take the MFMA kernels.
#include "common.hpp"
#include "internal.hpp"

#include <hip/hip_ext.h>
#include <math.h>

namespace bchip {

constexpr int F32_BLK = 32;      // list entries per block
constexpr int F32_SLOTS = 16;    // query slots a workgroup
constexpr int F32_THREADS = 256;

struct F32Params {
    const float* q;
    const float* kc;  // the row's cache (a ragged pool's offset applied)
    const float* vc;
    float* out;
    float* part_o;    // [unit][F32_SLOTS][HD]: chunk states of split launches
    float* part_ml;   // [unit][F32_SLOTS][2]
    const uint32_t* masks;
    uint32_t tree;
    uint32_t rows, nh, nkv, hd, G;
    uint32_t pos;     // line: slot of row 0; tree: the tree's first slot
    uint64_t slot_limit;  // slots the caches hold (tree slots past it read as zeros)
    float sc;         // scale * log2(e)
    uint32_t rb, nrb; // rows a workgroup (1 for trees), row blocks
    uint32_t nchunk;  // chunks of the farthest list
    uint32_t split;   // a workgroup per chunk
    const float* zero;  // ZERO_BYTES of zeros: the loads of rows past a list
    // A line call fused with RoPE and the K/V append of its rows at slots pos .. pos + rows - 1
    // (attn_f32<HD, NR, MS>, NR > 0: at most NR rows): q is unrotated on entry and rotated as it
    // is staged; the new K rows (knew, rotated here) and V rows (vnew) go to the caches and
    // stand in for those slots' cache entries. q is left rotated: by the workgroup itself when
    // unsplit, else by the fold.
    const float* knew;
    const float* vnew;
    const float* inv_freq;
    const uint32_t* positions;  // positions[r]: row r's rotation position
    uint32_t rope_dim, neox;
    float* qw;
};

// The dot's and P v's loops: two steps a trip at hd <= 64 (their LDS reads then go out
// together; configs[0]'s step 24.9 -> 22.7 us a layer), one at hd 128 (there the same
// measured slower, 76 -> 77-80 us: the registers cost more than the overlap gives).
template <int HD>
constexpr int F32_LU = HD <= 64 ? 2 : 1;

// Rows a fused line call of several rows takes (their K and V rows sit in LDS: at 8 rows and
// hd 128 three workgroups still fit a CU; 16 rows left two, and a verify pass's 704
// workgroups then took two turns of the GPU, 73 -> 96 us a layer-step).
constexpr uint32_t F32_FUSE_ROWS = 8;

template <int HD, int NR, bool MS>
__global__ __launch_bounds__(F32_THREADS) void attn_f32(const F32Params p) {
    constexpr bool FUSE = NR > 0;
    // q and K rows in LDS in lane order: element d = j + 8i at j * NI + i, so that the
    // elements of quant::dot's lane j (d = j, j + 8, ...) are contiguous and read 16 bytes at a
    // time. Rows are KS floats apart, 4 more than a multiple of 32 banks, so that the eight
    // lanes LDS serves together (eight entries, one offset) hit eight groups of banks.
    constexpr int NI = HD / 8;     // elements of one dot lane
    constexpr int KS = HD + 4;     // LDS row of q or K
    static_assert(NI % 4 == 0, "a lane's run is whole 16-byte reads");
    constexpr int NL = F32_BLK * (HD / 4) / F32_THREADS;  // 16-byte pieces of K (and of V) a thread loads a block
    static_assert(NL >= 1 && F32_BLK * (HD / 4) % F32_THREADS == 0, "a block's rows divide over the threads");
    // Each wave takes slots wave, wave + W, ...: their scores, softmax and P v within the wave.
    constexpr int W = F32_THREADS / 64;            // waves
    constexpr int SPW = F32_SLOTS / W;             // slots a wave at most
    constexpr int DPL = HD >= 64 ? HD / 64 : 1;    // dims a lane holds in P v
    constexpr int DL = HD / DPL;                   // lanes holding dims
    static_assert(F32_BLK == 32, "a block's entries are the wave's lanes 0..31");
    __shared__ __attribute__((aligned(16))) float qs[F32_SLOTS][KS];
    __shared__ __attribute__((aligned(16))) float ks[F32_BLK][KS];
    __shared__ __attribute__((aligned(16))) float vs[F32_BLK][HD];
    __shared__ uint32_t tail[MAX_ITEMS];
    // hd >= 128: each wave's P of a block (its slots of a pass), read back 16 bytes at a time for
    // the block sum and P v (eight reads a block where readlane took 32 VALU instructions:
    // configs[1] over f32 77.7 -> 75.5 us a call, its verify loop 70.8 -> 66.4 us a
    // layer-step; at hd 64 readlane measured slightly faster).
    constexpr bool PL = HD >= 128;
    constexpr int PS = MS ? F32_SLOTS / (F32_THREADS / 64) : 1;  // slots of a pass at most (one without MS)
    __shared__ __attribute__((aligned(16))) float pw[PL ? F32_THREADS / 64 : 1][PL ? PS : 1][PL ? F32_BLK : 4];
    // FUSE: the new K rows (rotated) and V rows as the caches hold them.
    __shared__ __attribute__((aligned(16))) float nrow[FUSE ? 2 : 1][FUSE ? NR : 1][FUSE ? HD : 4];

    const uint32_t tid = threadIdx.x;
    const uint32_t gi = p.split ? blockIdx.x / p.nchunk : blockIdx.x;
    const uint32_t c_one = p.split ? blockIdx.x % p.nchunk : 0u;
    const uint32_t kvh = gi % p.nkv;
    const uint32_t rbi = p.nrb - 1u - gi / p.nkv;  // latest rows (longest lists) first
    const uint32_t grp = kvh * p.nrb + rbi;        // canonical group of the chunk states
    const uint32_t r0 = rbi * p.rb;
    const uint32_t hd = p.hd, kvd = p.nkv * hd;
    const float* kcb = p.kc + (size_t)kvh * hd;
    const float* vcb = p.vc + (size_t)kvh * hd;

    // A tree's workgroup is one row: its list is the slots below pos, then pos + j for each
    // set bit j of its mask, in order (kernels.h:266-278).
    uint32_t ntail = 0;
    if (p.tree) {
        const uint32_t lo = p.masks[2 * r0], hi = p.masks[2 * r0 + 1];
        ntail = __popc(lo) + __popc(hi);
        if (tid < ntail) tail[tid] = p.pos + nth_set_bit(lo, hi, tid);
    }
    // Slot n: head kvh * G + n / rb of row r0 + n % rb.
    auto slot_valid = [&](uint32_t n) { return n / p.rb < p.G && r0 + n % p.rb < p.rows; };
    auto slot_len = [&](uint32_t n) -> uint32_t {
        if (!slot_valid(n)) return 0u;
        return p.tree ? p.pos + ntail : p.pos + r0 + n % p.rb + 1u;
    };
    const uint32_t rlast = min(r0 + p.rb, p.rows) - 1u;
    const uint32_t maxlen = p.tree ? p.pos + ntail : p.pos + rlast + 1u;
    // Slots at or past G * rb hold no query (a one-row step at G = 4 fills 4 of 16): the P v
    // products, the folds and the stores skip them, whole iterations at a time (uniform).
    const uint32_t used_e = min((uint32_t)F32_SLOTS, p.G * p.rb) * HD;


    const uint32_t lane = tid & 63u, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    // Slot wave + W s's running state: m, l, and the folded RM, RL (wave-uniform), and its
    // dims lane * DPL .. + DPL - 1 of o and R.
    float m[SPW], l[SPW], RM[SPW], RL[SPW], o[SPW][DPL], R[SPW][DPL];
#pragma unroll
    for (int s = 0; s < SPW; s++) {
        m[s] = RM[s] = -INFINITY;
        l[s] = RL[s] = 0.0f;
#pragma unroll
        for (int dd = 0; dd < DPL; dd++) o[s][dd] = R[s][dd] = 0.0f;
    }
    const uint32_t dl = lane % DL;  // this lane's dims in P v: dl * DPL .. (lanes past DL repeat them)

    // This thread's share of a block's K and V rows (NL 16-byte pieces of each), loaded one
    // block ahead: the next block's loads are in flight while this block computes. Entries
    // past the chunk or the cache, and dims past hd, load the zero page.
    f32x4 kr[NL], vr[NL];
    auto fetch = [&](uint32_t key0, uint32_t kb1) {
#pragma unroll
        for (int i = 0; i < NL; i++) {
            const uint32_t e = tid + F32_THREADS * i, k = e / (HD / 4), d = 4 * (e % (HD / 4)), kk = key0 + k;
            const uint32_t s = (p.tree && kk >= p.pos) ? tail[min(kk - p.pos, (uint32_t)MAX_ITEMS - 1u)] : kk;
            const bool ok = kk < kb1 && d < hd && (uint64_t)s < p.slot_limit;
            // One load each from a selected address (the asm keeps the compiler from
            // splitting it into a load on each side of a branch, each followed by a wait).
            uintptr_t ka = ok ? (uintptr_t)(kcb + (size_t)s * kvd + d) : (uintptr_t)p.zero;
            uintptr_t va = ok ? (uintptr_t)(vcb + (size_t)s * kvd + d) : (uintptr_t)p.zero;
            asm("" : "+v"(ka), "+v"(va));
            typedef __attribute__((address_space(1))) const f32x4 gf4;
            kr[i] = *(gf4*)ka;
            vr[i] = *(gf4*)va;
        }
    };
    auto stash = [&](uint32_t key0) {
#pragma unroll
        for (int i = 0; i < NL; i++) {
            const uint32_t e = tid + F32_THREADS * i, k = e / (HD / 4), d = 4 * (e % (HD / 4));
            f32x4 kx = kr[i], vx = vr[i];
            if constexpr (FUSE) {
                // A new row's slot: its K and V as this kernel wrote them to the caches.
                const uint32_t j = key0 + k - p.pos;
                if (key0 + k >= p.pos && j < p.rows) {
                    kx = *(const f32x4*)&nrow[0][j][d];
                    vx = *(const f32x4*)&nrow[1][j][d];
                }
            }
            float* kd = &ks[k][(d % 8) * NI + d / 8];  // d % 8 is 0 or 4: elements d .. d + 3 are lanes' runs apart
            kd[0] = kx[0];
            kd[NI] = kx[1];
            kd[2 * NI] = kx[2];
            kd[3 * NI] = kx[3];
            *(f32x4*)&vs[k][d] = vx;
        }
    };
    const uint32_t nused = used_e / HD;  // slots that may hold a query
    // Cross-lane moves: the value 32 lanes up; the max over 16- and 32-lane groups.
    auto up32 = [](float x) {
        return __uint_as_float(__builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false)[1]);
    };
    auto wave_max = [](float x) {
        x = fmaxf(x, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x128, 0xf, 0xf, false)));  // row_ror:8
        x = fmaxf(x, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x124, 0xf, 0xf, false)));  // row_ror:4
        x = fmaxf(x, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x122, 0xf, 0xf, false)));  // row_ror:2
        x = fmaxf(x, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x121, 0xf, 0xf, false)));  // row_ror:1
        const auto r16 = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
        x = fmaxf(__uint_as_float(r16[0]), __uint_as_float(r16[1]));
        const auto r32 = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
        return fmaxf(__uint_as_float(r32[0]), __uint_as_float(r32[1]));
    };

    // The first block's loads go out before q is staged, so that the two latencies overlap
    // (a tree's loads name slots from tail: every thread's entries of it are in first). Each
    // chunk's last block loads the next chunk's first (chunks past the list are empty, and
    // only they).
    if (p.tree) __syncthreads();
    const uint32_t cend = p.split ? c_one + 1u : max(1u, (maxlen + CHUNK_MULTI - 1u) / CHUNK_MULTI);
    if (c_one * CHUNK_MULTI < maxlen) fetch(c_one * CHUNK_MULTI, min(c_one * CHUNK_MULTI + CHUNK_MULTI, maxlen));
    if constexpr (FUSE) {
        // Row j's new slot is pos + j, its angles from positions[j]; pair pp of a head is (a, b)
        // by rope_pair, rotated when pp < rope_dim / 2 by k_rope_append's expressions (the
        // same bits).
        const size_t kvd_s = kvd;
        const uint32_t lo = max(c_one * CHUNK_MULTI, p.pos), hi = min(cend * CHUNK_MULTI, p.pos + p.rows);
        if (lo < hi) {
            // This workgroup streams new slots lo .. hi - 1: their K rows rotated and V rows,
            // into the caches and nrow (row blocks of the same chunk write the same values).
            for (uint32_t e = tid; e < (hi - lo) * (HD / 2); e += F32_THREADS) {
                const uint32_t j = lo - p.pos + e / (HD / 2), pp = e % (HD / 2);
                uint32_t a, b;
                const bool rot = rope_pair(pp, p.rope_dim, p.neox, a, b);
                float k0 = 0.0f, k1 = 0.0f, v0 = 0.0f, v1 = 0.0f;
                if (pp < hd / 2) {
                    const float* kx = p.knew + ((size_t)j * p.nkv + kvh) * hd;
                    const float* vx = p.vnew + ((size_t)j * p.nkv + kvh) * hd;
                    k0 = kx[a];
                    k1 = kx[b];
                    if (rot) rotate(kx[a], kx[b], (float)p.positions[j] * p.inv_freq[pp], k0, k1);
                    v0 = vx[2 * pp];
                    v1 = vx[2 * pp + 1];
                    float* kdst = (float*)p.kc + (size_t)(p.pos + j) * kvd_s + (size_t)kvh * hd;
                    float* vdst = (float*)p.vc + (size_t)(p.pos + j) * kvd_s + (size_t)kvh * hd;
                    kdst[a] = k0;
                    kdst[b] = k1;
                    vdst[2 * pp] = v0;
                    vdst[2 * pp + 1] = v1;
                }
                nrow[0][j][a] = k0;
                nrow[0][j][b] = k1;
                nrow[1][j][2 * pp] = v0;
                nrow[1][j][2 * pp + 1] = v1;
            }
        }
        // q rotated as it is staged, a pair a thread (dims past hd and empty slots: zeros).
        for (uint32_t e = tid; e < F32_SLOTS * (HD / 2); e += F32_THREADS) {
            const uint32_t n = e / (HD / 2), pp = e % (HD / 2);
            uint32_t a, b;
            const bool rot = rope_pair(pp, p.rope_dim, p.neox, a, b);
            float y0 = 0.0f, y1 = 0.0f;
            if (pp < hd / 2 && slot_valid(n)) {
                const uint32_t r = r0 + n % p.rb, h = kvh * p.G + n / p.rb;
                const float* qh = p.q + ((size_t)r * p.nh + h) * hd;
                y0 = qh[a];
                y1 = qh[b];
                if (rot) rotate(qh[a], qh[b], (float)p.positions[r] * p.inv_freq[pp], y0, y1);
            }
            qs[n][(a % 8) * NI + a / 8] = y0;
            qs[n][(b % 8) * NI + b / 8] = y1;
        }
        if (!p.split) {
            // q stays rotated, as k_rope_append leaves it: this workgroup is the only reader of
            // its heads, and every read of them is done at the barrier. (A split launch's fold
            // writes them once every chunk's workgroup has read them.)
            __syncthreads();
            for (uint32_t e = tid; e < F32_SLOTS * HD; e += F32_THREADS) {
                const uint32_t n = e / HD, d = e % HD;
                if (d < hd && slot_valid(n)) {
                    const uint32_t r = r0 + n % p.rb, h = kvh * p.G + n / p.rb;
                    p.qw[((size_t)r * p.nh + h) * hd + d] = qs[n][(d % 8) * NI + d / 8];
                }
            }
        }
    } else {
        for (uint32_t e = tid; e < F32_SLOTS * HD; e += F32_THREADS) {
            const uint32_t n = e / HD, d = e % HD;
            float v = 0.0f;
            if (d < hd && slot_valid(n)) {
                const uint32_t r = r0 + n % p.rb, h = kvh * p.G + n / p.rb;
                v = p.q[((size_t)r * p.nh + h) * hd + d];
            }
            qs[n][(d % 8) * NI + d / 8] = v;
        }
    }
    for (uint32_t c = c_one; c < cend; c++) {
        const uint32_t kb0 = c * CHUNK_MULTI, kb1 = min(kb0 + CHUNK_MULTI, maxlen);
        for (uint32_t key0 = kb0; key0 < kb1; key0 += F32_BLK) {
            __syncthreads();  // the previous block's K, V and P are consumed (and q is in)
            stash(key0);
            if (key0 + F32_BLK < kb1) {
                fetch(key0 + F32_BLK, kb1);
            } else if (c + 1 < cend && kb1 < maxlen) {
                const uint32_t nb0 = (c + 1) * CHUNK_MULTI;
                fetch(nb0, min(nb0 + CHUNK_MULTI, maxlen));
            }
            // K and V in for everyone. The fences order LDS only: __syncthreads' would also
            // wait for the next block's loads just issued.
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
            __builtin_amdgcn_s_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
            // Per slot of this wave: scores, softmax and P v. Lane k < 32 and lane k + 32 take
            // entry k: each sums quant::dot's lanes 4h .. 4h + 3 (h its half) over their
            // elements in order, and lane k adds the eight to 0 in lane order (the upper four
            // from lane k + 32), times sc; -inf at or past the slot's list. The block's max
            // across the wave; P of entry k in lane k; the block sum and P v entry by entry
            // in order, P taken from its lane.
            const uint32_t k = lane & 31u, h = lane >> 5;
            // Slots s0 .. s0 + NS - 1 of the wave together: each slot's operations as alone,
            // in the same order; K's and V's LDS reads serve all of them.
            auto pass = [&](auto S0, auto NSc) {
                constexpr int s0 = decltype(S0)::value, NS = decltype(NSc)::value;
                static_assert(s0 + NS <= SPW && (!PL || NS <= PS), "a pass's slots are the wave's, its P rows in pw");
                uint32_t nn[NS];
                float a[NS][4];
#pragma unroll
                for (int s = 0; s < NS; s++) {
                    nn[s] = wave + W * (s0 + s);
#pragma unroll
                    for (int jj = 0; jj < 4; jj++) a[s][jj] = 0.0f;
                }
                // d = j + 8 (i + t) in order; past hd (a head dim below HD) no term.
                auto dot_lanes = [&](auto FULL) {
#pragma unroll F32_LU<HD>
                    for (uint32_t i = 0; i < (uint32_t)NI; i += 4) {
#pragma unroll
                        for (uint32_t jj = 0; jj < 4; jj++) {
                            const uint32_t j = 4 * h + jj;
                            const f32x4 kv = *(const f32x4*)&ks[k][j * NI + i];
#pragma unroll
                            for (int s = 0; s < NS; s++) {
                                const f32x4 qv = *(const f32x4*)&qs[nn[s]][j * NI + i];
#pragma unroll
                                for (uint32_t t = 0; t < 4; t++)
                                    if (decltype(FULL)::value || 8 * (i + t) < hd) a[s][jj] += qv[t] * kv[t];
                            }
                        }
                    }
                };
                if (hd == (uint32_t)HD)
                    dot_lanes(std::true_type{});
                else
                    dot_lanes(std::false_type{});
                float pe[NS], mn[NS], cr[NS];
#pragma unroll
                for (int s = 0; s < NS; s++) {
                    float dsum = 0.0f + a[s][0];
                    dsum += a[s][1];
                    dsum += a[s][2];
                    dsum += a[s][3];
#pragma unroll
                    for (int jj = 0; jj < 4; jj++) dsum += up32(a[s][jj]);
                    const float sc = (lane < 32u && key0 + k < slot_len(nn[s])) ? dsum * p.sc : -INFINITY;
                    const float mx = wave_max(sc);
                    mn[s] = fmaxf(m[s0 + s], mx);
                    const float ms = (mn[s] == -INFINITY) ? 0.0f : mn[s];
                    cr[s] = exp2_hw(m[s0 + s] - ms);
                    pe[s] = exp2_hw(sc - ms);
                }
                float bl[NS], acc[NS][DPL];
                if constexpr (PL) {
#pragma unroll
                    for (int s = 0; s < NS; s++)
                        if (lane < 32u) pw[wave][s][lane] = pe[s];
                }
#pragma unroll
                for (int s = 0; s < NS; s++) {
                    bl[s] = 0.0f;
#pragma unroll
                    for (int dd = 0; dd < DPL; dd++) acc[s][dd] = 0.0f;
                }
#pragma unroll F32_LU<HD>
                for (int k8 = 0; k8 < F32_BLK; k8 += 8) {
                    f32x4 pq[NS][2];
                    if constexpr (PL) {
#pragma unroll
                        for (int s = 0; s < NS; s++) {
                            pq[s][0] = *(const f32x4*)&pw[wave][s][k8];
                            pq[s][1] = *(const f32x4*)&pw[wave][s][k8 + 4];
                        }
                    }
#pragma unroll
                    for (int kj = 0; kj < 8; kj++) {
                        const int kk = k8 + kj;
                        float v[DPL];
                        if constexpr (DPL == 1) {
                            v[0] = vs[kk][dl];
                        } else if constexpr (DPL == 2) {
                            const float2 v2 = *(const float2*)&vs[kk][2 * dl];
                            v[0] = v2.x;
                            v[1] = v2.y;
                        } else {
                            const f32x4 v4 = *(const f32x4*)&vs[kk][4 * dl];
#pragma unroll
                            for (int dd = 0; dd < 4; dd++) v[dd] = v4[dd];
                        }
#pragma unroll
                        for (int s = 0; s < NS; s++) {
                            const float pk = PL ? pq[s][kj / 4][kj % 4]
                                                : __int_as_float(__builtin_amdgcn_readlane(__float_as_int(pe[s]), kk));
                            bl[s] += pk;
#pragma unroll
                            for (int dd = 0; dd < DPL; dd++) acc[s][dd] += pk * v[dd];
                        }
                    }
                }
#pragma unroll
                for (int s = 0; s < NS; s++) {
                    l[s0 + s] = l[s0 + s] * cr[s] + bl[s];
                    m[s0 + s] = mn[s];
#pragma unroll
                    for (int dd = 0; dd < DPL; dd++) o[s0 + s][dd] = o[s0 + s][dd] * cr[s] + acc[s][dd];
                }
            };
            using i0 = std::integral_constant<int, 0>;
            using i1 = std::integral_constant<int, 1>;
            using i2 = std::integral_constant<int, 2>;
            using i3 = std::integral_constant<int, 3>;
            static_assert(SPW == 4, "four slots a wave at most");
            // The wave's slots that may hold a query: wave, wave + W, ... below nused.
            const uint32_t nact = wave < nused ? min((uint32_t)SPW, (nused - wave + W - 1) / W) : 0u;
            if constexpr (MS && HD > 64) {
                // A launch whose waves hold several slots (MS: more than four in a workgroup):
                // four a pass where a wave has four, else two.
                if (nact == 4) {
                    pass(i0{}, std::integral_constant<int, 4>{});
                } else {
                    if (nact >= 2)
                        pass(i0{}, i2{});
                    else if (nact == 1)
                        pass(i0{}, i1{});
                    if (nact == 3) pass(i2{}, i1{});
                }
            } else if constexpr (HD <= 64) {
                // Two slots a pass: the shared reads and the two slots' chains side by side
                // (configs[0], seven slots over four waves: 22.7 -> 21.9 us a layer-step).
                if (nact >= 2)
                    pass(i0{}, i2{});
                else if (nact == 1)
                    pass(i0{}, i1{});
                if (nact >= 4)
                    pass(i2{}, i2{});
                else if (nact == 3)
                    pass(i2{}, i1{});
            } else {
                if (nact >= 1) pass(i0{}, i1{});
                if (nact >= 2) pass(i1{}, i1{});
                if (nact >= 3) pass(i2{}, i1{});
                if (nact >= 4) pass(i3{}, i1{});
            }
        }
        if (p.split) break;
        // The chunk's state folded into the running one (merge_coef, R = R a + c b).
#pragma unroll
        for (int sw = 0; sw < SPW; sw++) {
            float fa, fb, mn;
            merge_coef(RM[sw], m[sw], fa, fb, mn);
            RL[sw] = RL[sw] * fa + l[sw] * fb;
            RM[sw] = mn;
#pragma unroll
            for (int dd = 0; dd < DPL; dd++) {
                R[sw][dd] = R[sw][dd] * fa + o[sw][dd] * fb;
                o[sw][dd] = 0.0f;
            }
            m[sw] = -INFINITY;
            l[sw] = 0.0f;
        }
    }
    if (p.split) {
        const size_t u = (size_t)grp * p.nchunk + c_one;
#pragma unroll
        for (int sw = 0; sw < SPW; sw++) {
            const uint32_t n = wave + W * sw;
            if (n >= nused) break;  // attn_combine reads no slot past them
            if (lane < (uint32_t)DL) {
#pragma unroll
                for (int dd = 0; dd < DPL; dd++) p.part_o[(u * F32_SLOTS + n) * HD + DPL * dl + dd] = o[sw][dd];
            }
            if (lane == 0) *(float2*)(p.part_ml + (u * F32_SLOTS + n) * 2) = float2{m[sw], l[sw]};
        }
        return;
    }
#pragma unroll
    for (int sw = 0; sw < SPW; sw++) {
        const uint32_t n = wave + W * sw;
        if (n >= nused) break;
        if (!slot_valid(n) || lane >= (uint32_t)DL) continue;
        const uint32_t r = r0 + n % p.rb, hh = kvh * p.G + n / p.rb;
#pragma unroll
        for (int dd = 0; dd < DPL; dd++) {
            const uint32_t d = DPL * dl + dd;
            if (d < hd) p.out[((size_t)r * p.nh + hh) * hd + d] = R[sw][dd] / RL[sw];
        }
    }
}

static uint32_t ceil_div32(uint64_t a, uint64_t b) { return (uint32_t)((a + b - 1) / b); }

template <int HD, bool MS>
static void launch_f32_ms(const F32Params& fp, uint32_t blocks, const AttnCall& a, hipStream_t s, bool fuse) {
    if (fuse && fp.rows == 1)
        hipExtLaunchKernelGGL((attn_f32<HD, 1, MS>), dim3(blocks), dim3(F32_THREADS), 0, s, a.ev_before, a.ev_after, 0,
                              fp);
    else if (fuse)
        hipExtLaunchKernelGGL((attn_f32<HD, (int)F32_FUSE_ROWS, MS>), dim3(blocks), dim3(F32_THREADS), 0, s,
                              a.ev_before, a.ev_after, 0, fp);
    else
        hipExtLaunchKernelGGL((attn_f32<HD, 0, MS>), dim3(blocks), dim3(F32_THREADS), 0, s, a.ev_before, a.ev_after, 0,
                              fp);
}

// MS: a launch whose workgroups hold more than four query slots (a wave then has several);
// its own kernels, so that the one-slot-a-wave step keeps the registers of one pass.
template <int HD>
static hipError_t launch_f32_t(const F32Params& fp, uint32_t blocks, const AttnCall& a, hipStream_t s, bool fuse) {
    if constexpr (HD > 64) {
        if (fp.G * fp.rb > (uint32_t)(F32_THREADS / 64)) {
            launch_f32_ms<HD, true>(fp, blocks, a, s, fuse);
            return hipGetLastError();
        }
    }
    launch_f32_ms<HD, false>(fp, blocks, a, s, fuse);
    return hipGetLastError();
}

hipError_t f32_attention(const AttnCall& a, uint64_t kvoff, Workspace& ws, hipStream_t s, const RopeArgs* rope) {
    if (a.rows == 0 || a.nkv == 0 || a.nh % a.nkv != 0 || a.hd == 0 || a.hd % 8 != 0 || a.hd > MAX_HD)
        return hipErrorInvalidValue;
    if (a.tree && a.rows > MAX_ITEMS) return hipErrorInvalidValue;
    if (rope && (a.tree || a.rows > F32_FUSE_ROWS || kvoff != 0 || rope->rope_dim % 2 || rope->rope_dim > a.hd))
        return hipErrorInvalidValue;
    F32Params fp{};
    if (rope) {
        fp.knew = rope->k;
        fp.vnew = rope->v;
        fp.inv_freq = rope->inv_freq;
        fp.positions = rope->positions;
        fp.rope_dim = rope->rope_dim;
        fp.neox = rope->neox;
        fp.qw = rope->q;
    }
    const uint64_t kvd = (uint64_t)a.nkv * a.hd;
    fp.q = a.q;
    fp.kc = (const float*)a.kc + kvoff * kvd;
    fp.vc = (const float*)a.vc + kvoff * kvd;
    fp.out = a.out;
    fp.masks = a.masks;
    fp.tree = a.tree;
    fp.rows = a.rows;
    fp.nh = a.nh;
    fp.nkv = a.nkv;
    fp.hd = a.hd;
    fp.G = a.nh / a.nkv;
    if (fp.G > (uint32_t)F32_SLOTS) return hipErrorInvalidValue;
    fp.pos = a.pos;
    fp.slot_limit = a.slot_limit > kvoff ? a.slot_limit - kvoff : 0;
    fp.zero = (const float*)ws.zero;
    fp.sc = a.scale * LOG2E;
    fp.rb = a.tree ? 1u : std::max<uint32_t>(1u, (uint32_t)F32_SLOTS / fp.G);
    if (fp.rb > a.rows) fp.rb = a.rows;
    fp.nrb = ceil_div32(a.rows, fp.rb);
    // A tree row's list reaches at most 64 entries past pos (its mask's bits); a line's
    // longest is its last row's.
    const uint64_t far = a.tree ? (uint64_t)a.pos + MAX_ITEMS : (uint64_t)a.pos + a.rows;
    fp.nchunk = ceil_div32(far, CHUNK_MULTI);
    const uint64_t groups = (uint64_t)a.nkv * fp.nrb;
    fp.split = groups < 512 && fp.nchunk > 1;
    const uint32_t hdp = a.hd <= 32 ? 32u : a.hd <= 64 ? 64u : a.hd <= 128 ? 128u : 256u;
    if (fp.split) {
        hipError_t e = ws.reserve((size_t)groups * fp.nchunk * F32_SLOTS, hdp);
        if (e == hipSuccess) {
            fp.part_o = ws.o;
            fp.part_ml = ws.ml;
        } else if (ws.fixed) {
            fp.split = 0;  // a fixed workspace too small for the states: unsplit, the same bits
        } else {
            return e;
        }
    }
    const uint64_t blocks = groups * (fp.split ? fp.nchunk : 1u);
    if (blocks > 0x7fffffffull) return hipErrorInvalidValue;
    hipError_t e;
    switch (hdp) {
        case 32: e = launch_f32_t<32>(fp, (uint32_t)blocks, a, s, rope != nullptr); break;
        case 64: e = launch_f32_t<64>(fp, (uint32_t)blocks, a, s, rope != nullptr); break;
        case 128: e = launch_f32_t<128>(fp, (uint32_t)blocks, a, s, rope != nullptr); break;
        default: e = launch_f32_t<256>(fp, (uint32_t)blocks, a, s, rope != nullptr); break;
    }
    if (e != hipSuccess || !fp.split) return e;
    CombineParams cp{};
    cp.long_fold = ws.combine_long;
    cp.zero = ws.zero;
    cp.out = a.out;
    cp.part_o = ws.o;
    cp.part_ml = ws.ml;
    cp.nh = a.nh;
    cp.nkv = a.nkv;
    cp.hd = a.hd;
    cp.G = fp.G;
    cp.slots = F32_SLOTS;
    cp.slots_out = F32_SLOTS;
    cp.shared = 1;
    cp.rows = a.rows;
    cp.rb = fp.rb;
    cp.nrb = fp.nrb;
    cp.nchunk = fp.nchunk;
    if (rope) {
        cp.fuse = 1;
        cp.qw = rope->q;
        cp.inv_freq = rope->inv_freq;
        cp.positions = rope->positions;
        cp.rope_dim = rope->rope_dim;
        cp.neox = rope->neox;
    }
    return combine_launch(cp, (uint32_t)groups, a.hd, s);
}

}  // namespace bchip
