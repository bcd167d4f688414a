// Internal interface between the C ABI (bchip.hip) and the kernel files.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "common.hpp"

namespace bchip {

// Device scratch for split-K partials, owned by a context and grown on demand; or, fixed,
// a view of memory set aside once (the no-allocation entry point's): then a reserve beyond
// it fails with hipErrorOutOfMemory and nothing is allocated.
struct Workspace {
    float* o = nullptr;    // [units*slots][hd_pad]: chunk states
    float* ml = nullptr;   // [units*slots][2]
    void* zero = nullptr;  // ZERO_BYTES of zeros
    // Arrival counters of the single-launch folds (GROUP_COUNTERS, GROUP_STRIDE words apart,
    // zero between calls), the device's CU count (how many one-CU workgroups can be resident
    // at once), and a word in host memory that a fold whose wait ran out sets (never
    // otherwise): bchip_sync reports it.
    uint32_t* gcnt = nullptr;
    uint32_t cus = 0;
    // BCHIP_GROUP_FOLD at init: 0 turns the single-launch folds off; "spread" makes every
    // group take the path of a group spread over several XCDs (for tests of that path).
    // BCHIP_GROUP_FOLD_SPINS bounds their waits (for tests of a wait that runs out).
    bool group_fold = true;
    uint32_t group_spread = 0;
    uint32_t group_spins = 1u << 16;
    // BCHIP_COMBINE_LONG=0 at init: lists of more than CMB_RUN chunks fold in attn_combine
    // as shorter ones do, not in attn_combine_long (the same bits; for tests).
    bool combine_long = true;
    // BCHIP_ROW_RUNS at init: one-row launches give each unit a run of chunks when they have
    // many units (1, the default), always (2) or never (0); the same bits (for tests).
    uint32_t row_runs = 1;
    uint32_t* gerr = nullptr;       // device address of the host word
    volatile uint32_t* gerr_host = nullptr;
    void* vt = nullptr;    // V^T tiles of a prefill call; the sampler's keys and sort scratch
    float* qrot = nullptr;  // rotated q of a fused step, until attn_row_fold copies it
    size_t slots = 0, hdp = 0, vt_bytes = 0, qrot_floats = 0;
    bool fixed = false;
    size_t o_cap = 0, ml_cap = 0, qrot_cap = 0;  // fixed: bytes of o, ml and qrot
    hipError_t init(int device);  // allocates the zero page, the counters and the error word
    // The fixed view: o, ml and qrot at base (o_bytes, ml_bytes, q_bytes each); the zero page,
    // counters and error word of `owner`.
    void set_fixed(void* base, size_t o_bytes, size_t ml_bytes, size_t q_bytes, const Workspace& owner);
    hipError_t reserve(size_t need_slots, size_t hd_pad);
    hipError_t reserve_qrot(size_t floats);
    hipError_t reserve_vt(size_t bytes);
    void release();
};

constexpr size_t ZERO_BYTES = 4096;
constexpr uint32_t GROUP_COUNTERS = 1024;
constexpr uint32_t GROUP_STRIDE = 32;  // one 128-byte line a counter

struct AttnCall {
    const float* q;
    const void* kc;
    const void* vc;
    uint32_t kv_type;  // 0 f32, 1 f16
    float* out;
    const uint32_t* masks;
    uint32_t tree, rows, nh, nkv, hd, pos;
    float scale;
    uint64_t slot_limit;  // slots both caches hold (all slots a call may read when unknown)
    // Timing: when set, recorded at the start and the end of the call's main attention
    // kernel by its dispatch (hipExtLaunchKernel), not the V^T pack before it nor the fold
    // or combine after it.
    hipEvent_t ev_before = nullptr, ev_after = nullptr;
};

// One-row items (row, len, kvoff): decode steps and ragged batches, one launch.
hipError_t row_attention(const AttnCall& a, const Item* items, uint32_t nitems, Workspace& ws, hipStream_t s);
// A one-row step fused with k_rope(q), k_rope(k) and the K/V append at slot a.pos (the row's
// last visible slot): q is rotated (and left rotated), k and v (f32 [nkv][hd]) go into the
// caches. Requires hd % 32 == 0 and, for neox pairs, rope_dim/2 % 32 == 0.
struct RopeArgs {
    float* q;
    const float* k;
    const float* v;
    const float* inv_freq;
    const uint32_t* positions;
    uint32_t rope_dim, neox;
};
hipError_t row_attention_fused(const AttnCall& a, const RopeArgs& r, Workspace& ws, hipStream_t s);
// Several sequences' fused steps in one launch: item i is row items[i].row of q, k, v, out and
// positions, its cache at items[i].kvoff with items[i].len slots, the new row the last.
hipError_t row_attention_fused_items(const AttnCall& a, const RopeArgs& r, const Item* items, uint32_t nitems,
                                     Workspace& ws, hipStream_t s);
bool row_fusable(uint32_t nh, uint32_t nkv, uint32_t hd, uint32_t rope_dim, uint32_t neox);
// Workspace slots (chunk states) a one-row call over a list of len entries takes.
size_t row_state_slots(uint64_t len, uint32_t nkv);
// Tree rows as items with chunk and nchunk set (CHUNK_MULTI).
hipError_t direct_attention(const AttnCall& a, const Item* items, uint32_t nitems,
                            Workspace& ws, hipStream_t s);
hipError_t shared_attention(const AttnCall& a, Workspace& ws, hipStream_t s);
// A line of rows (verify) with RoPE and the K/V append of its rows (slots pos + r) in the
// same launch: the bits of rope_append_launch then shared_attention. hipErrorNotSupported
// (nothing launched) where the plan is not a split pass folded in its launch of f16 hd-128
// caches of at most FUSE_ROWS rows: the caller then makes the two calls.
hipError_t shared_attention_fused(const AttnCall& a, const RopeArgs& r, Workspace& ws, hipStream_t s);
// The left fold of chunk states (attn_combine) over `groups` groups of cp.
hipError_t combine_launch(CombineParams& cp, uint32_t groups, uint32_t hd, hipStream_t s);
// Every call on an f32 cache (lines, trees, one row): f32 arithmetic throughout
// (attention_f32.hip). kvoff: slot offset of the row's cache in a ragged pool. rope (a line
// call of at most 8 rows, kvoff 0): the call fused with RoPE and the K/V append of its rows
// at slots a.pos .., the bits of rope_append_launch then f32_attention.
hipError_t f32_attention(const AttnCall& a, uint64_t kvoff, Workspace& ws, hipStream_t s,
                         const RopeArgs* rope = nullptr);

hipError_t rope_launch(float* x, const float* inv_freq, const uint32_t* positions, uint32_t rows,
                       uint32_t heads, uint32_t hd, uint32_t rope_dim, uint32_t neox, hipStream_t s);
hipError_t rope_append_launch(float* q, const float* k, const float* v, void* kc, void* vc, uint32_t kv_type,
                              const float* inv_freq, const uint32_t* positions, uint32_t rows, uint32_t nh,
                              uint32_t nkv, uint32_t hd, uint32_t rope_dim, uint32_t neox, uint64_t slot0,
                              hipStream_t s);
// Row r of q, k, v to cache slot slots[r] (host array): one new row of each of several
// sequences in one pool.
hipError_t rope_append_ragged_launch(float* q, const float* k, const float* v, void* kc, void* vc, uint32_t kv_type,
                                     const float* inv_freq, const uint32_t* positions, uint32_t rows, uint32_t nh,
                                     uint32_t nkv, uint32_t hd, uint32_t rope_dim, uint32_t neox,
                                     const uint64_t* slots, hipStream_t s);
hipError_t copy_launch(const void* src, uint32_t st, void* dst, uint32_t dt, uint64_t off, uint64_t n, hipStream_t s);
hipError_t move_launch(void* buf, uint32_t type, uint64_t from, uint64_t to, uint64_t n, hipStream_t s);
hipError_t keep_launch(void* const* bufs, uint32_t nbufs, uint32_t type, uint32_t width, uint64_t base,
                       const uint32_t* rows, uint32_t nrows, hipStream_t s);
hipError_t grow_launch(const void* const* src, void* const* dst, uint32_t nbufs, uint64_t keep_bytes,
                       uint64_t total_bytes, hipStream_t s);
hipError_t fill_normal_launch(void* dst, uint32_t type, uint64_t n, uint64_t seed, hipStream_t s);

// The sampler (sample.hip): ids[r] = sample.rs's pick for row r of scores [rows][vocab] at step
// step0 + r. scratch: sample_scratch_bytes(rows, vocab) bytes (unused for temperature <= 0).
size_t sample_scratch_bytes(uint32_t rows, uint32_t vocab);
hipError_t sample_launch(const float* scores, uint32_t rows, uint32_t vocab, float temperature, float top_p,
                         uint64_t seed, uint64_t step0, uint32_t* ids, void* scratch, size_t scratch_bytes,
                         hipStream_t s);

// The rest of a layer (layer.hip).
bool ggml_block(uint32_t type, uint32_t& weights, uint32_t& bytes);
// Input rows one product call takes: passes of 8 rows over the grid's y dimension (65535).
constexpr uint32_t MATMUL_MAX_N = 8u * 65535u;
// Batches of n >= 2 input rows of the quantised formats and F16 (cols a multiple of 256)
// run on the matrix cores; their K splits may need matmul_scratch_bytes of scratch (partial
// sums) and a context's MATMUL_COUNTERS arrival counters (zero when no product runs).
constexpr uint32_t MATMUL_COUNTERS = 1024;
bool matmul_uses_mm(uint32_t type, uint32_t cols, uint32_t n);
size_t matmul_scratch_bytes(uint32_t type, uint32_t rows, uint32_t cols, uint32_t n);
hipError_t matmul_launch(const void* w, uint32_t type, const float* x, float* out, uint32_t rows, uint32_t cols,
                         uint32_t n, uint32_t row_bytes, void* scratch, uint32_t* counters, hipStream_t s);
hipError_t rms_norm_launch(const float* x, const float* w, float* out, uint32_t rows, uint32_t cols, float eps,
                           bool vec, hipStream_t s);
enum : int { EW_BIAS = 0, EW_SILU_MUL = 1, EW_ADD = 2 };
hipError_t elementwise_launch(int op, float* x, const float* y, uint64_t n, uint32_t dim, hipStream_t s);

}  // namespace bchip
