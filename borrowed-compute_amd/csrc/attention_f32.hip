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
};

template <int HD>
__global__ __launch_bounds__(F32_THREADS) void attn_f32(const F32Params p) {
    constexpr int NP = F32_SLOTS * HD / F32_THREADS;  // (slot, dim) outputs a thread
    static_assert(NP >= 1 && (F32_SLOTS * HD) % F32_THREADS == 0, "outputs divide over the threads");
    // q and K rows in LDS in lane order: element d = j + 8i at j * JS + i, so that score lane
    // j's elements (d = j, j + 8, ...) are contiguous and read 16 bytes at a time; JS pads a
    // lane's run so that the eight lanes of an entry read eight distinct groups of banks.
    constexpr int NI = HD / 8;                    // elements a score lane takes
    constexpr int JS = NI % 8 == 0 ? NI + 4 : NI;  // LDS stride between lanes' runs
    constexpr int KS = 8 * JS;                    // LDS row of q or K
    static_assert(NI % 4 == 0, "a lane's run is whole 16-byte reads");
    constexpr int NL = F32_BLK * (HD / 4) / F32_THREADS;  // 16-byte pieces of K (and of V) a thread loads a block
    static_assert(NL >= 1 && F32_BLK * (HD / 4) % F32_THREADS == 0, "a block's rows divide over the threads");
    __shared__ __attribute__((aligned(16))) float qs[F32_SLOTS][KS];
    __shared__ __attribute__((aligned(16))) float ks[F32_BLK][KS];
    __shared__ __attribute__((aligned(16))) float vs[F32_BLK][HD];
    __shared__ __attribute__((aligned(16))) float ps[F32_SLOTS][F32_BLK + 4];  // rows 16-byte aligned
    __shared__ float corr_s[F32_SLOTS], fa[F32_SLOTS], fb[F32_SLOTS], lsum[F32_SLOTS];
    __shared__ uint32_t tail[MAX_ITEMS];

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

    for (uint32_t e = tid; e < F32_SLOTS * HD; e += F32_THREADS) {
        const uint32_t n = e / HD, d = e % HD;
        float v = 0.0f;
        if (d < hd && slot_valid(n)) {
            const uint32_t r = r0 + n % p.rb, h = kvh * p.G + n / p.rb;
            v = p.q[((size_t)r * p.nh + h) * hd + d];
        }
        qs[n][(d % 8) * JS + d / 8] = v;
    }

    float o[NP], R[NP];
#pragma unroll
    for (int i = 0; i < NP; i++) o[i] = R[i] = 0.0f;
    // Slot n's running state: m in lanes 4n .. 4n + 3 of wave 0 (the softmax's lanes of the
    // slot), l, RM and RL in lane 4n.
    float m = -INFINITY, l = 0.0f, RM = -INFINITY, RL = 0.0f;
    const bool slot_lane = tid < 4u * F32_SLOTS && (tid & 3u) == 0u;
    const uint32_t sn = tid >> 2;  // the slot of a softmax lane

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
    auto stash = [&]() {
#pragma unroll
        for (int i = 0; i < NL; i++) {
            const uint32_t e = tid + F32_THREADS * i, k = e / (HD / 4), d = 4 * (e % (HD / 4));
            float* kd = &ks[k][(d % 8) * JS + d / 8];  // d % 8 is 0 or 4: elements d .. d + 3 are lanes' runs apart
            kd[0] = kr[i][0];
            kd[JS] = kr[i][1];
            kd[2 * JS] = kr[i][2];
            kd[3 * JS] = kr[i][3];
            *(f32x4*)&vs[k][d] = vr[i];
        }
    };
    // Scores: slot by slot, thread (entry qk, lane qj) sums q[d] k[d] over d = qj, qj + 8, ...
    // in order (quant::dot's lane qj), and lane 0 of each eight adds the eight sums to 0 in
    // lane order (row shifts within the 16-lane row).
    const uint32_t qk = tid >> 3, qj = tid & 7;
    const uint32_t nused = used_e / HD;  // slots that may hold a query

    const uint32_t cend = p.split ? c_one + 1u : max(1u, (maxlen + CHUNK_MULTI - 1u) / CHUNK_MULTI);
    for (uint32_t c = c_one; c < cend; c++) {
        const uint32_t kb0 = c * CHUNK_MULTI, kb1 = min(kb0 + CHUNK_MULTI, maxlen);
        if (kb0 < kb1) fetch(kb0, kb1);
        for (uint32_t key0 = kb0; key0 < kb1; key0 += F32_BLK) {
            __syncthreads();  // the previous block's K, V and P are consumed (and q is in)
            stash();
            if (key0 + F32_BLK < kb1) fetch(key0 + F32_BLK, kb1);
            // K and V in for everyone. The fences order LDS only: __syncthreads' would also
            // wait for the next block's loads just issued.
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
            __builtin_amdgcn_s_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
            // Scores of (slot, entry) pairs: quant::dot's eight lane sums, then times sc;
            // entries at or past a slot's list are -inf.
            // Two slots at a time (each K value read once for both; a slot past nused computes
            // on zeros and is not written); the lane's steps unrolled over HD, so its LDS reads
            // go out ahead of the sums that take them.
            auto lane_sum = [&](float acc) {  // lane 0 of each eight: 0 + acc_0 + ... + acc_7
                const int ai = __float_as_int(acc);
                float dsum = 0.0f + acc;
                dsum += __int_as_float(__builtin_amdgcn_update_dpp(0, ai, 0x101, 0xf, 0xf, false));
                dsum += __int_as_float(__builtin_amdgcn_update_dpp(0, ai, 0x102, 0xf, 0xf, false));
                dsum += __int_as_float(__builtin_amdgcn_update_dpp(0, ai, 0x103, 0xf, 0xf, false));
                dsum += __int_as_float(__builtin_amdgcn_update_dpp(0, ai, 0x104, 0xf, 0xf, false));
                dsum += __int_as_float(__builtin_amdgcn_update_dpp(0, ai, 0x105, 0xf, 0xf, false));
                dsum += __int_as_float(__builtin_amdgcn_update_dpp(0, ai, 0x106, 0xf, 0xf, false));
                dsum += __int_as_float(__builtin_amdgcn_update_dpp(0, ai, 0x107, 0xf, 0xf, false));
                return dsum;
            };
            for (uint32_t n = 0; n < nused; n += 2) {
                float acc0 = 0.0f, acc1 = 0.0f;
#pragma unroll
                for (uint32_t i = 0; i < (uint32_t)NI; i += 4) {
                    const f32x4 kv = *(const f32x4*)&ks[qk][qj * JS + i];
                    const f32x4 q0 = *(const f32x4*)&qs[n][qj * JS + i];
                    const f32x4 q1 = *(const f32x4*)&qs[n + 1][qj * JS + i];
#pragma unroll
                    for (uint32_t t = 0; t < 4; t++) {
                        if (8 * (i + t) < hd) {  // d = qj + 8 (i + t) in order; past hd nothing
                            acc0 += q0[t] * kv[t];
                            acc1 += q1[t] * kv[t];
                        }
                    }
                }
                const float s0 = lane_sum(acc0), s1 = lane_sum(acc1);
                if (qj == 0) {
                    ps[n][qk] = (key0 + qk < slot_len(n)) ? s0 * p.sc : -INFINITY;
                    if (n + 1 < nused) ps[n + 1][qk] = (key0 + qk < slot_len(n + 1)) ? s1 * p.sc : -INFINITY;
                }
            }
            for (uint32_t e = nused * F32_BLK + tid; e < F32_SLOTS * F32_BLK; e += F32_THREADS)
                ps[e / F32_BLK][e % F32_BLK] = -INFINITY;
            __syncthreads();
            // Per slot: the block's max, the new running max, P and the block's sum of P.
            // Lanes 4n .. 4n + 3 of wave 0 take slot n's entries eight each: the block's max
            // across the four (a max is exact in any order), P in parallel, and the block's
            // sum in entry order by lane 4n (its own eight, then the others' from LDS).
            static_assert(F32_BLK == 32 && 4 * F32_SLOTS == 64, "wave 0 holds every slot's softmax");
            if (tid < 4u * F32_SLOTS) {
                const uint32_t k0 = 8 * (tid & 3u);
                f32x4 pa = *(const f32x4*)&ps[sn][k0], pb = *(const f32x4*)&ps[sn][k0 + 4];
                float mx = fmaxf(fmaxf(fmaxf(pa[0], pa[1]), fmaxf(pa[2], pa[3])), fmaxf(fmaxf(pb[0], pb[1]), fmaxf(pb[2], pb[3])));
                mx = fmaxf(mx, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(mx), 0xB1, 0xf, 0xf, false)));
                mx = fmaxf(mx, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(mx), 0x4E, 0xf, 0xf, false)));
                const float mn = fmaxf(m, mx), ms = (mn == -INFINITY) ? 0.0f : mn;
                const float cr = exp2_hw(m - ms);
#pragma unroll
                for (int t = 0; t < 4; t++) {
                    pa[t] = exp2_hw(pa[t] - ms);
                    pb[t] = exp2_hw(pb[t] - ms);
                }
                *(f32x4*)&ps[sn][k0] = pa;
                *(f32x4*)&ps[sn][k0 + 4] = pb;
                if ((tid & 3u) == 0u) {
                    float bl = 0.0f;
#pragma unroll
                    for (int t = 0; t < 4; t++) bl += pa[t];
#pragma unroll
                    for (int t = 0; t < 4; t++) bl += pb[t];
#pragma unroll
                    for (int k = 8; k < F32_BLK; k += 4) {
                        const f32x4 c = *(const f32x4*)&ps[sn][k];
                        bl += c[0];
                        bl += c[1];
                        bl += c[2];
                        bl += c[3];
                    }
                    l = l * cr + bl;
                    corr_s[sn] = cr;
                }
                m = mn;
            }
            __syncthreads();
            // O = O * corr + sum of P v, the sum in entry order.
#pragma unroll
            for (int i = 0; i < NP; i++) {
                const uint32_t e = tid + F32_THREADS * i, n = e / HD, d = e % HD;
                if (F32_THREADS * i >= used_e) break;
                float acc = 0.0f;
                for (int k = 0; k < F32_BLK; k++) acc += ps[n][k] * vs[k][d];
                o[i] = o[i] * corr_s[n] + acc;
            }
        }
        if (p.split) break;
        // The chunk's state folded into the running one (merge_coef, R = R a + c b).
        if (slot_lane) {
            float a, b, mn;
            merge_coef(RM, m, a, b, mn);
            RL = RL * a + l * b;
            RM = mn;
            fa[sn] = a;
            fb[sn] = b;
        }
        m = -INFINITY;
        l = 0.0f;
        __syncthreads();
#pragma unroll
        for (int i = 0; i < NP; i++) {
            const uint32_t n = (tid + F32_THREADS * i) / HD;
            if (F32_THREADS * i >= used_e) break;
            R[i] = R[i] * fa[n] + o[i] * fb[n];
            o[i] = 0.0f;
        }
        __syncthreads();  // fa and fb are read before the next chunk's fold writes them
    }
    if (p.split) {
        const size_t u = (size_t)grp * p.nchunk + c_one;
#pragma unroll
        for (int i = 0; i < NP; i++) {
            const uint32_t e = tid + F32_THREADS * i, n = e / HD, d = e % HD;
            if (F32_THREADS * i >= used_e) break;  // attn_combine reads no slot past them
            p.part_o[(u * F32_SLOTS + n) * HD + d] = o[i];
        }
        if (slot_lane) *(float2*)(p.part_ml + (u * F32_SLOTS + sn) * 2) = float2{m, l};
        return;
    }
    if (slot_lane) lsum[sn] = RL;
    __syncthreads();
#pragma unroll
    for (int i = 0; i < NP; i++) {
        const uint32_t e = tid + F32_THREADS * i, n = e / HD, d = e % HD;
        if (d < hd && slot_valid(n)) {
            const uint32_t r = r0 + n % p.rb, h = kvh * p.G + n / p.rb;
            p.out[((size_t)r * p.nh + h) * hd + d] = R[i] / lsum[n];
        }
    }
}

static uint32_t ceil_div32(uint64_t a, uint64_t b) { return (uint32_t)((a + b - 1) / b); }

template <int HD>
static hipError_t launch_f32_t(const F32Params& fp, uint32_t blocks, const AttnCall& a, hipStream_t s) {
    hipExtLaunchKernelGGL((attn_f32<HD>), dim3(blocks), dim3(F32_THREADS), 0, s, a.ev_before, a.ev_after, 0, fp);
    return hipGetLastError();
}

hipError_t f32_attention(const AttnCall& a, uint64_t kvoff, Workspace& ws, hipStream_t s) {
    if (a.rows == 0 || a.nkv == 0 || a.nh % a.nkv != 0 || a.hd == 0 || a.hd % 8 != 0 || a.hd > MAX_HD)
        return hipErrorInvalidValue;
    if (a.tree && a.rows > MAX_ITEMS) return hipErrorInvalidValue;
    F32Params fp{};
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
        case 32: e = launch_f32_t<32>(fp, (uint32_t)blocks, a, s); break;
        case 64: e = launch_f32_t<64>(fp, (uint32_t)blocks, a, s); break;
        case 128: e = launch_f32_t<128>(fp, (uint32_t)blocks, a, s); break;
        default: e = launch_f32_t<256>(fp, (uint32_t)blocks, a, s); break;
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
    return combine_launch(cp, (uint32_t)groups, a.hd, s);
}

}  // namespace bchip
