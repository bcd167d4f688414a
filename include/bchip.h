/* bchip: bc-infer's attention path on one AMD Instinct MI355X (gfx950), as a C ABI.
 *
 * This is the boundary a `gpu/hip.rs` backend binds in place of `gpu/cuda.rs`
 * (crates/bc-infer/src/gpu/cuda.rs:1-95) for the attention sub-sequence of
 * `Layers::forward` (crates/bc-infer/src/gpu/mod.rs:464-482), `Cache::keep`
 * (mod.rs:322-337) and `Layers::reserve` (mod.rs:404-423). Plain pointers and sizes only.
 *
 * Conventions
 *  - Every call returns an int: BCHIP_OK (0) or a negative BCHIP_E_* code; the message of
 *    the last failing call on this thread is bchip_last_error(). Nothing aborts or throws
 *    across the ABI (the reference maps failures to anyhow::Result, gpu/mod.rs:119-134).
 *  - "Device pointer" arguments are addresses in the context's device memory, from
 *    bchip_alloc or any other allocator on that device. Host pointers are only read or
 *    written during the call.
 *  - All kernels run in order on the context's one stream (cuda.rs:40, one stream);
 *    launches return before the work ends; bchip_sync waits (cuda.rs:93). The caller
 *    serialises calls on one context, as the reference's Gpu mutex does (mod.rs:105-107).
 *  - Element types of cache buffers: BCHIP_F32 (the reference's f32 cache, mod.rs:409-421)
 *    or BCHIP_F16 (IEEE binary16, rounded to nearest even: new with this backend).
 *  - Cache layout is the reference's: per layer, K and V each [slots][n_head_kv*head_dim]
 *    (slot t of KV head h at t*kvd + h*head_dim, mod.rs:473-475, kernels.h:287,310).
 */
#ifndef BCHIP_H
#define BCHIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define BCHIP_ABI_VERSION 6

enum bchip_type { BCHIP_F32 = 0, BCHIP_F16 = 1 }; /* T_F32 / T_F16 of kernels.h:14-15 */

enum bchip_status {
    BCHIP_OK = 0,
    BCHIP_E_ARG = -1,         /* an argument is out of range or inconsistent */
    BCHIP_E_HIP = -2,         /* the HIP runtime reported an error */
    BCHIP_E_NODEV = -3,       /* no usable gfx950 device */
    BCHIP_E_DISABLED = -4,    /* BC_INFER_GPU=0 in the environment (mod.rs:116) */
    BCHIP_E_UNSUPPORTED = -5, /* a shape this backend does not take */
    BCHIP_E_OOM = -6          /* device memory exhausted */
};

typedef struct bchip_ctx bchip_ctx;

/* Message of the last failing call on this thread ("" if none). */
const char* bchip_last_error(void);
int bchip_abi_version(void);

/* Backend::new (cuda.rs:32-42): opens `device`, checks it is gfx950, creates the stream.
 * Fails with BCHIP_E_DISABLED when BC_INFER_GPU=0 (gpu/mod.rs:116). */
int bchip_init(int device, bchip_ctx** ctx);
int bchip_destroy(bchip_ctx* ctx);

/* Backend::name (cuda.rs:44-46): NUL-terminated, truncated to len. */
int bchip_device_name(bchip_ctx* ctx, char* buf, size_t len);
/* Backend::memory (cuda.rs:49-51): free device bytes now. */
int bchip_mem_free(bchip_ctx* ctx, uint64_t* free_bytes);
/* Backend::unified (cuda.rs:53-55): 0, memory is the card's own. */
int bchip_unified(bchip_ctx* ctx, int* unified);

/* Backend::zeros (cuda.rs:66-68): `bytes` of zeroed device memory (at least 1). */
int bchip_alloc(bchip_ctx* ctx, size_t bytes, void** dev);
/* Drop of a Buf (cudarc frees on drop). */
int bchip_free(bchip_ctx* ctx, void* dev);
/* Backend::upload / weights (cuda.rs:57-64): host -> dev+off, synchronous. */
int bchip_upload(bchip_ctx* ctx, void* dev, size_t off, const void* host, size_t bytes);
/* Backend::read (cuda.rs:70-76): dev+off -> host after all queued work, synchronous. */
int bchip_download(bchip_ctx* ctx, const void* dev, size_t off, void* host, size_t bytes);
/* The wait at the end of Backend::run (cuda.rs:93). */
int bchip_sync(bchip_ctx* ctx);
/* The context's hipStream_t (for callers that time or order their own work on it). */
int bchip_stream(bchip_ctx* ctx, void** hip_stream);

/* k_rope (kernels.h:237-248, entry cuda.cu:81; launched at mod.rs:464-472): rotates, in
 * place, pair i of every head of row r of x [rows][heads][hd] (f32) by
 * positions[r] * inv_freq[i]; neox pairs (i, i + rope_dim/2), else (2i, 2i+1).
 * positions: device u32 [rows]; inv_freq: device f32 [rope_dim/2]. */
int bchip_rope(bchip_ctx* ctx, float* x, const float* inv_freq, const uint32_t* positions,
               uint32_t rows, uint32_t heads, uint32_t hd, uint32_t rope_dim, uint32_t neox);

/* k_copy (kernels.h:332, entry cuda.cu:90; mod.rs:413-420, 473-475):
 * dst[dst_off + i] = src[i] for i < n (element offsets and counts), converting from
 * src_type to dst_type (f32 -> f16 rounds to nearest even). */
int bchip_copy(bchip_ctx* ctx, const void* src, uint32_t src_type, void* dst,
               uint32_t dst_type, uint64_t dst_off, uint64_t n);

/* k_move (kernels.h:334, entry cuda.cu:89): within one buffer, b[to + i] = b[from + i]
 * for i < n elements, to <= from; overlapping ranges are handled. */
int bchip_move(bchip_ctx* ctx, void* buf, uint32_t type, uint64_t from, uint64_t to, uint64_t n);

/* Cache::keep (mod.rs:322-337) for `nbufs` cache buffers at once (every layer's K and V):
 * row base+rows[i] moves to base+i for each i with rows[i] != i, in order. rows (host) must
 * ascend (Kv::keep's check, model.rs:147); nrows <= 64. width = n_head_kv * head_dim.
 * bufs is a host array of device pointers. */
int bchip_keep(bchip_ctx* ctx, void* const* bufs, uint32_t nbufs, uint32_t type, uint32_t width,
               uint64_t base, const uint32_t* rows, uint32_t nrows);

/* The copy step of Gpu::reserve (mod.rs:404-423): for each of `nbufs` pairs (every layer's
 * K and V), dst[0, keep) = src[0, keep) and dst[keep, total) = 0, in elements of `type`,
 * all pairs in one launch (the reference zero-allocates each new buffer, then issues one
 * K::Copy per buffer). src and dst are host arrays of device pointers, each 16-byte
 * aligned; a pair's ranges may not overlap; src may be NULL when keep is 0. */
int bchip_cache_grow(bchip_ctx* ctx, const void* const* src, void* const* dst, uint32_t nbufs, uint32_t type,
                     uint64_t keep, uint64_t total);

/* The attention sub-sequence k_rope(q), k_rope(k), k_copy(k -> kc), k_copy(v -> vc)
 * (mod.rs:464-475) as one launch: rotates q [rows][nh][hd] in place, rotates k
 * [rows][nkv][hd] and writes it, with v [rows][nkv][hd], into cache slots slot0 + r of
 * kc and vc (type kv_type). k and v (f32) are read only. positions as bchip_rope. */
int bchip_rope_append(bchip_ctx* ctx, float* q, const float* k, const float* v, void* kc, void* vc,
                      uint32_t kv_type, const float* inv_freq, const uint32_t* positions,
                      uint32_t rows, uint32_t nh, uint32_t nkv, uint32_t hd, uint32_t rope_dim,
                      uint32_t neox, uint64_t slot0);

/* k_attention (kernels.h:250-324, entry cuda.cu:82-85; launched at mod.rs:476-482):
 * causal grouped-query attention of `rows` rows. q, out: device f32 [rows][nh][hd];
 * kc, vc: cache of kv_type; head h reads KV head h / (nh/nkv).
 *  - tree == 0 (a line): row r sees slots 0 .. pos + r.
 *  - tree != 0: pos is the tree's first slot; row r sees slots 0 .. pos-1 and the slots
 *    pos + j for each set bit j of its 64-bit mask, masks[2r] (bits 0-31) and
 *    masks[2r+1] (bits 32-63) (device u32 [2*rows], mod.rs:436-442), summed in list order:
 *    the k-th entry of the list is slot k below pos, then the (k-pos)-th set bit
 *    (kernels.h:266-278), so a tree row gets exactly the bits of the line its path is.
 *     A tree grown a level at a time holds more nodes than the pass has rows (Shape::new,
 *    model.rs:421-443), so a mask may name any slot up to pos + 63: the caches must hold
 *    every slot the masks name (the caller's Shape guarantees it; in a bchip_alloc buffer a
 *    slot past its end reads as zeros, never out of bounds). rows <= 64, pos + 64 <= 2^32.
 * Requires hd % 8 == 0, hd <= 256, nh % nkv == 0, nh/nkv <= 16.
 * f32 caches (the reference's): f32 arithmetic throughout, the scores by quant::dot's
 * eight-lane sum (quant.rs:617-631), one arithmetic for every row of every call: a row's
 * bits depend only on its q and its visible slot list, whatever the batch, the row's index,
 * tree or line, one row or many (model.rs:531, 578, 592-594, 641-646).
 * f16 caches: q, K, V and the softmax weights are f16 MFMA operands, f32 accumulation.
 * Every row of a multi-row call (rows >= 2) is computed by the same fixed-order
 * arithmetic, which depends only on the row's q and its visible slot list: results are
 * identical whatever the batch, the row's index, or whether it is a tree node or a line
 * token. A one-row call (a decode step) cuts its list into at most 256 chunks (their length
 * set by the list length and nkv alone) and folds the chunk states in a fixed order:
 * deterministic, and within rounding of the same row in a batch (the reference allows
 * 1e-4, model.rs:641-642). */
int bchip_attention(bchip_ctx* ctx, const float* q, const void* kc, const void* vc,
                    uint32_t kv_type, float* out, const uint32_t* masks, uint32_t tree,
                    uint32_t rows, uint32_t nh, uint32_t nkv, uint32_t hd, uint32_t pos,
                    float scale);

/* One decode step of one layer as a single call: bchip_rope_append with rows = 1 and
 * slot0 = pos, then bchip_attention with rows = 1, tree = 0 at pos, with the same results
 * bit for bit (out; q left rotated; the new row in kc and vc). It is the peephole over the
 * five commands k_rope(q), k_rope(k), k_copy(k), k_copy(v), k_attention that
 * Layers::forward queues per layer for a one-token pass (gpu/mod.rs:464-482): the rotation
 * and the append run inside the attention kernel, which takes the new row from registers
 * (f16 caches) or LDS (f32 caches: attn_f32 rotates q as it stages it and the fold leaves q
 * rotated). f16 shapes the fused kernel does not take (hd % 32 != 0, neox pairs with
 * rope_dim/2 not a multiple of 32, or more than 8 query heads per KV head) run as the two
 * calls. positions: device u32 [1]. */
int bchip_rope_append_attention(bchip_ctx* ctx, float* q, const float* k, const float* v, void* kc, void* vc,
                                uint32_t kv_type, const float* inv_freq, const uint32_t* positions, uint32_t nh,
                                uint32_t nkv, uint32_t hd, uint32_t rope_dim, uint32_t neox, uint32_t pos,
                                float scale, float* out);

/* One layer of a multi-row pass (a speculative verify step, llm.rs:655-667; a chain of
 * draft rows) as a single call: bchip_rope_append with slot0 = pos, then bchip_attention
 * (tree = 0) of the same rows at pos, with the same results bit for bit (out; q left
 * rotated; rows r of k and v in slots pos + r of kc and vc). It is the peephole over the
 * commands k_rope(q), k_rope(k), k_copy(k), k_copy(v), k_attention that Layers::forward
 * queues per layer for a pass of several rows (gpu/mod.rs:464-482). One launch does the
 * rotations, the appends and the attention (its workgroups take the new rows from LDS) for
 * f16 caches at head_dim 128, at most 16 rows with rows x (nh / nkv) <= 64, a line longer
 * than one 192-slot chunk whose split launch fits the device's CUs at once, neox pairs
 * only at rope_dim 64 or 128, and k and v 16-byte aligned; and for f32 caches of at most 8
 * rows at any shape (attn_f32, then its fold when split). Other calls run as the two calls.
 * positions: device u32 [rows]. */
int bchip_rope_append_attention_rows(bchip_ctx* ctx, float* q, const float* k, const float* v, void* kc, void* vc,
                                     uint32_t kv_type, const float* inv_freq, const uint32_t* positions,
                                     uint32_t rows, uint32_t nh, uint32_t nkv, uint32_t hd, uint32_t rope_dim,
                                     uint32_t neox, uint32_t pos, float scale, float* out);

/* bchip_rope_append_attention that allocates nothing. It has no counterpart in the
 * reference; it is for callers that cannot allocate device memory mid-run (code under HIP
 * graph capture, tight serving loops, harnesses that forbid allocation). Same arguments and
 * the same results, bit for bit. Its scratch (a step's chunk states and the staged rotated q)
 * is a fixed array in device memory, one copy per device from the library's load until the
 * process ends: 16 MiB of chunk states (a one-row plan of at most 1024 units x 16 slots x 256
 * dims: any plan with n_head_kv <= 1024), 128 KiB of their maxima and sums, 256 KiB of q
 * (nh * hd <= 65536 for the fused kernel). A step that needs more is refused with BCHIP_E_ARG
 * before anything is launched; an f32 cache never needs more (its pass then runs unsplit, the
 * same bits). Every call on one device shares that array, so calls on one device that overlap
 * in time (from several contexts, threads or streams) race. */
int bchip_rope_append_attention_noalloc(bchip_ctx* ctx, float* q, const float* k, const float* v, void* kc,
                                        void* vc, uint32_t kv_type, const float* inv_freq,
                                        const uint32_t* positions, uint32_t nh, uint32_t nkv, uint32_t hd,
                                        uint32_t rope_dim, uint32_t neox, uint32_t pos, float scale, float* out);

/* Several conversations' one-token steps in one launch (the reference runs one
 * k_attention per KV stream, crates/bc-mesh/src/engine.rs:25,305-309): sequence i's row
 * q[i] [nh][hd] sees the seq_lens[i] slots kv_offsets[i] .. kv_offsets[i]+seq_lens[i]-1 of
 * the shared kc/vc pool (a ragged layout). Each sequence's result equals bchip_attention
 * with rows = 1, pos = seq_lens[i]-1 on its own slots, bit for bit. seq_lens and
 * kv_offsets are host arrays; nseq <= 256. Not for graph capture across calls with
 * different lengths: the plan is made on the host from seq_lens. */
int bchip_attention_ragged(bchip_ctx* ctx, const float* q, const void* kc, const void* vc,
                           uint32_t kv_type, float* out, const uint32_t* seq_lens,
                           const uint64_t* kv_offsets, uint32_t nseq, uint32_t nh,
                           uint32_t nkv, uint32_t hd, float scale);

/* The append of one new row to each of several conversations in one cache pool, as one
 * launch (the reference keeps up to 16 conversations' caches a stage and appends each with
 * its own k_rope and k_copy, crates/bc-mesh/src/engine.rs:25, 305-314, gpu/mod.rs:464-475):
 * sequence i's q row [nh][hd] and k row [nkv][hd] turn by positions[i] (device u32 [nseq];
 * normally seq_lens[i] - 1), and k and v go into slot kv_offsets[i] + seq_lens[i] - 1 of kc and
 * vc, its last visible slot. seq_lens, kv_offsets: host arrays; nseq <= 256; sequences' slots
 * must not overlap. Each row's bits are those of bchip_rope_append with rows = 1 at that slot. */
int bchip_rope_append_ragged(bchip_ctx* ctx, float* q, const float* k, const float* v, void* kc, void* vc,
                             uint32_t kv_type, const float* inv_freq, const uint32_t* positions,
                             const uint32_t* seq_lens, const uint64_t* kv_offsets, uint32_t nseq, uint32_t nh,
                             uint32_t nkv, uint32_t hd, uint32_t rope_dim, uint32_t neox);

/* One decode step of several conversations: bchip_rope_append_ragged, then
 * bchip_attention_ragged over the same seq_lens and kv_offsets, with the same results bit for
 * bit; for f16 caches and the shapes bchip_rope_append_attention fuses, one launch does the
 * rotations, the appends and the attention of every sequence (at most 64 a launch). */
int bchip_rope_append_attention_ragged(bchip_ctx* ctx, float* q, const float* k, const float* v, void* kc,
                                       void* vc, uint32_t kv_type, const float* inv_freq,
                                       const uint32_t* positions, const uint32_t* seq_lens,
                                       const uint64_t* kv_offsets, uint32_t nseq, uint32_t nh, uint32_t nkv,
                                       uint32_t hd, uint32_t rope_dim, uint32_t neox, float scale, float* out);

/* ---- The rest of a layer (Layers::forward, mod.rs:454-491): the GGUF block-format
 * product, RMSNorm and the elementwise ops. Weight types are ggml's numbers
 * (quant.rs:35-49): BCHIP_GGML_F32 0, F16 1, Q4_0 2, Q4_1 3, Q5_0 6, Q5_1 7, Q8_0 8,
 * Q4K 12, Q5K 13, Q6K 14, BF16 30. */
#define BCHIP_GGML_F32 0u
#define BCHIP_GGML_F16 1u
#define BCHIP_GGML_Q4_0 2u
#define BCHIP_GGML_Q4_1 3u
#define BCHIP_GGML_Q5_0 6u
#define BCHIP_GGML_Q5_1 7u
#define BCHIP_GGML_Q8_0 8u
#define BCHIP_GGML_Q4K 12u
#define BCHIP_GGML_Q5K 13u
#define BCHIP_GGML_Q6K 14u
#define BCHIP_GGML_BF16 30u

/* k_matmul (kernels.h:189-214, entry cuda.cu:77-79; Gpu::matmul / matmul_rows,
 * gpu/mod.rs:158-178): out[i][r] = sum_c W[r][c] x[i][c] for i < n, r < rows. w holds the
 * weight matrix as stored (rows of whole ggml blocks of `type`, row stride
 * cols / block_weights * block_bytes: matmul_rows passes its first `rows` rows only);
 * x [n][cols] and out [n][rows] f32. cols must be a multiple of 32 (256 for the K-quants);
 * w and x 16-byte aligned; n at most 524280 (8 x 65535) a call. Batches of 2 or more rows
 * of the block formats and F16 with cols a multiple of 256 run on the matrix cores, as the
 * reference's do from MM_FROM = 2 rows (gpu/mod.rs:33-41). An input row's result does not
 * depend on n or on its place among the batch's rows; a batch row agrees with the same row
 * passed alone within f32 rounding (as the reference's). Reruns give the same bits. */
int bchip_matmul(bchip_ctx* ctx, const void* w, uint32_t type, const float* x, float* out,
                 uint32_t rows, uint32_t cols, uint32_t n);

/* k_rms_norm (kernels.h:216-225, entry cuda.cu:80; mod.rs:455, 485): for each of rows
 * rows of cols, out = x / sqrt(mean(x^2) + eps) * w (w [cols]). */
int bchip_rms_norm(bchip_ctx* ctx, const float* x, const float* w, float* out, uint32_t rows,
                   uint32_t cols, float eps);

/* k_bias_add (kernels.h:328, entry cuda.cu:86; mod.rs:459-463): x[i] += b[i % dim], i < n. */
int bchip_bias_add(bchip_ctx* ctx, float* x, const float* b, uint64_t n, uint32_t dim);

/* k_silu_mul (kernels.h:329, entry cuda.cu:87; mod.rs:488): g[i] = g[i] / (1 + e^-g[i]) * u[i]. */
int bchip_silu_mul(bchip_ctx* ctx, float* g, const float* u, uint64_t n);

/* k_add (kernels.h:330, entry cuda.cu:88; mod.rs:484, 490): x[i] += y[i], i < n. */
int bchip_add(bchip_ctx* ctx, float* x, const float* y, uint64_t n);

/* sample.rs:24-71 on the device, the step after the logits head (gpu/mod.rs:499-508;
 * engine.rs:341-350): ids[r] (device u32 [rows]) = the token picked from row r of scores
 * (device f32 [rows][vocab]) at step step0 + r. temperature <= 0: the first index of the
 * highest score. Otherwise p = exp((score - max) / temperature) (exp correctly rounded: the
 * reference takes its C library's expf, equal but for arguments within 0.002 ulp of a rounding
 * midpoint), the smallest prefix of the stable descending order whose mass reaches top_p, and
 * the seeded draw of sample.rs:61-67 with uniform(seed ^ step * 0x9e3779b97f4a7c15). Every sum
 * runs in the reference's order, so the ids are the reference's. rows <= 65535. */
int bchip_sample(bchip_ctx* ctx, const float* scores, uint32_t rows, uint32_t vocab, float temperature,
                 float top_p, uint64_t seed, uint64_t step0, uint32_t* ids);

/* Seeded N(0,1) draws into dst (n elements of type): splitmix64 (Steele, Lea and Flood
 * 2014) + Box-Muller (1958), the generator of the benchmark inputs; draw i of seed s is
 * the oracle's draw i of s up to the last bit of the device's log/sin/cos. */
int bchip_fill_normal(bchip_ctx* ctx, void* dst, uint32_t type, uint64_t n, uint64_t seed);

/* Timing on the context's stream: start records an event; stop records another, waits
 * for it and returns the milliseconds between them. */
int bchip_timer_start(bchip_ctx* ctx);
int bchip_timer_stop(bchip_ctx* ctx, float* ms);
/* Arms the next attention call (bchip_attention, bchip_attention_ragged,
 * bchip_rope_append_attention) to record the caller's HIP events `before` and `after`
 * (hipEvent_t) at the start and the end of its main attention kernel, by that kernel's
 * dispatch (hipExtLaunchKernel), leaving out the V^T pack before it and the fold or combine
 * after it: the duration of the dominant kernel as a kernel trace reports it. One call
 * consumes the arming. */
int bchip_timer_arm(bchip_ctx* ctx, void* before, void* after);

#ifdef __cplusplus
}
#endif
#endif
