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
};

template <int HD>
__global__ __launch_bounds__(F32_THREADS) void attn_f32(const F32Params p) {
    constexpr int QS = HD + 1;                         // LDS row stride of q and K: rows on distinct banks
    constexpr int NP = F32_SLOTS * HD / F32_THREADS;  // (slot, dim) outputs a thread
    static_assert(NP >= 1 && (F32_SLOTS * HD) % F32_THREADS == 0, "outputs divide over the threads");
    __shared__ float qs[F32_SLOTS][QS];
    __shared__ float ks[F32_BLK][QS];
    __shared__ __attribute__((aligned(16))) float vs[F32_BLK][HD];
    __shared__ float ps[F32_SLOTS][F32_BLK + 1];
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
        qs[n][d] = v;
    }

    float o[NP], R[NP];
#pragma unroll
    for (int i = 0; i < NP; i++) o[i] = R[i] = 0.0f;
    float m = -INFINITY, l = 0.0f, RM = -INFINITY, RL = 0.0f;  // slot threads (tid < F32_SLOTS)

    const uint32_t cend = p.split ? c_one + 1u : max(1u, (maxlen + CHUNK_MULTI - 1u) / CHUNK_MULTI);
    for (uint32_t c = c_one; c < cend; c++) {
        const uint32_t kb0 = c * CHUNK_MULTI, kb1 = min(kb0 + CHUNK_MULTI, maxlen);
        for (uint32_t key0 = kb0; key0 < kb1; key0 += F32_BLK) {
            __syncthreads();  // the previous block's K, V and P are consumed (and q is in)
            for (uint32_t e = tid; e < F32_BLK * (HD / 4); e += F32_THREADS) {
                const uint32_t k = e / (HD / 4), d = 4 * (e % (HD / 4)), kk = key0 + k;
                float4 kv = float4{0.0f, 0.0f, 0.0f, 0.0f}, vv = kv;
                if (kk < kb1 && d < hd) {
                    const uint32_t s = (p.tree && kk >= p.pos) ? tail[kk - p.pos] : kk;
                    if ((uint64_t)s < p.slot_limit) {
                        kv = *(const float4*)(kcb + (size_t)s * kvd + d);
                        vv = *(const float4*)(vcb + (size_t)s * kvd + d);
                    }
                }
                ks[k][d] = kv.x;
                ks[k][d + 1] = kv.y;
                ks[k][d + 2] = kv.z;
                ks[k][d + 3] = kv.w;
                *(float4*)&vs[k][d] = vv;
            }
            __syncthreads();
            // Scores of (slot, entry) pairs: quant::dot's eight lane sums, then times sc;
            // entries at or past a slot's list are -inf.
            for (uint32_t e = tid; e < F32_SLOTS * F32_BLK; e += F32_THREADS) {
                const uint32_t n = e / F32_BLK, k = e % F32_BLK;
                float s = -INFINITY;
                if (key0 + k < slot_len(n)) {
                    float acc[8] = {0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
                    for (uint32_t d = 0; d < hd; d += 8) {
#pragma unroll
                        for (int j = 0; j < 8; j++) acc[j] += qs[n][d + j] * ks[k][d + j];
                    }
                    float dsum = 0.0f;
#pragma unroll
                    for (int j = 0; j < 8; j++) dsum += acc[j];
                    s = dsum * p.sc;
                }
                ps[n][k] = s;
            }
            __syncthreads();
            // Per slot: the block's max, the new running max, P and the block's sum of P.
            if (tid < (uint32_t)F32_SLOTS) {
                float mx = -INFINITY;
                for (int k = 0; k < F32_BLK; k++) mx = fmaxf(mx, ps[tid][k]);
                const float mn = fmaxf(m, mx), ms = (mn == -INFINITY) ? 0.0f : mn;
                const float cr = exp2_hw(m - ms);
                float bl = 0.0f;
                for (int k = 0; k < F32_BLK; k++) {
                    const float pe = exp2_hw(ps[tid][k] - ms);
                    ps[tid][k] = pe;
                    bl += pe;
                }
                l = l * cr + bl;
                m = mn;
                corr_s[tid] = cr;
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
        if (tid < (uint32_t)F32_SLOTS) {
            float a, b, mn;
            merge_coef(RM, m, a, b, mn);
            RL = RL * a + l * b;
            RM = mn;
            fa[tid] = a;
            fb[tid] = b;
            m = -INFINITY;
            l = 0.0f;
        }
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
        if (tid < (uint32_t)F32_SLOTS) *(float2*)(p.part_ml + (u * F32_SLOTS + tid) * 2) = float2{m, l};
        return;
    }
    if (tid < (uint32_t)F32_SLOTS) lsum[tid] = RL;
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
