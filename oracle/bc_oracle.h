/* CPU oracle for bc-infer's attention path: TEST INFRASTRUCTURE, NOT PRODUCT CODE.
 *
 * A plain-C restatement of the reference's f32 CPU attention path, used only by tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg, as the checker. The product
 * (libbchip.so) never links, loads or calls anything here.
 *
 * Every function names the reference lines it follows (paths relative to the
 * Harshil089/Borrowed-Compute checkout):
 *   bco_inv_freq   crates/bc-infer/src/model.rs:208-211
 *   bco_rope       crates/bc-infer/src/model.rs:391-403
 *   bco_shape      crates/bc-infer/src/model.rs:405-443 (ROOT, MAX_TREE, Shape::new)
 *   bco_dot        crates/bc-infer/src/quant.rs:617-631
 *   bco_attention  crates/bc-infer/src/model.rs:445-481
 *   bco_keep       crates/bc-infer/src/model.rs:146-166 (Kv::keep on one cache buffer)
 *   bco_f16_*      IEEE binary16 round-to-nearest-even, the rounding the GPU's f16 KV
 *                  cache applies (the reference's own f32_to_f16, quant.rs:113-131,
 *                  rounds half-up and flushes subnormals: test-fixture grade only)
 *   bco_normal     splitmix64 (Steele, Lea and Flood 2014) + Box-Muller (1958) N(0,1)
 *                  draws, the seeded input generator of the benchmark configurations
 *
 * Parity pinning (each function is checked by tests/test_oracle.py against an
 * independent derivation, not a retyped formula): f64 brute force and torch's
 * scaled_dot_product_attention in f64 for bco_attention; closed forms (one key, equal
 * keys, constant values, a dominant key) and invariants (key-permutation, GQA equals MHA
 * with replicated heads); the reference's own rope test (model.rs:676-688) and rotation
 * invariants for bco_rope; exhaustive small trees and the reference's tree test shape
 * (model.rs:561-611) for bco_shape and bco_keep; numpy float16 for bco_f16_*; the
 * published splitmix64 output sequence for bco_normal's generator.
 */
#ifndef BC_ORACLE_H
#define BC_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* A tree row that follows the cached text directly (model.rs:406). */
#define BCO_ROOT 0xffffffffu
/* Rows a tree pass may hold (model.rs:408). */
#define BCO_MAX_TREE 64

/* inv_freq[i] = base^(-2i/rope_dim) / factors[i] (factors may be NULL), i < rope_dim/2. */
void bco_inv_freq(float* out, uint32_t rope_dim, float base, const float* factors);

/* Rotates every head of one row (heads x head_dim floats, in place) to position pos. */
void bco_rope(float* x, uint32_t heads, uint32_t head_dim, uint32_t rope_dim, int neox,
              uint64_t pos, const float* inv_freq);

/* Where each of `rows` rows sits and what it sees. tree == NULL is a line. On success
 * writes positions[rows], and for a tree visible[rows] (bit j = slot base + j) and *base;
 * returns 0, or -1 for a tree Shape::new rejects. */
int bco_shape(uint32_t rows, uint64_t pos, const uint32_t* tree, uint32_t tree_len,
              uint64_t* positions, uint64_t* visible, uint64_t* base);

/* Sum of a[i]*b[i] in 8 lane accumulators, then the remainder, in the reference order. */
float bco_dot(const float* a, const float* b, size_t n);

/* Causal grouped-query attention of `rows` rows at positions pos.. against the cache:
 * q [rows][nh][hd], kc/vc [slots][nkv*hd], out [rows][nh][hd]. With visible != NULL
 * (a tree from slot base), row i sees slots 0..base and base+j for bit j of visible[i];
 * else slots 0..pos+i. scale multiplies every dot product (the reference uses
 * 1/sqrt(hd)). */
void bco_attention(const float* q, const float* kc, const float* vc, float* out,
                   uint32_t rows, uint64_t pos, const uint64_t* visible, uint64_t base,
                   uint32_t nh, uint32_t nkv, uint32_t hd, float scale);

/* Kv::keep on one cache buffer of `*len` rows of `width` floats: moves rows base+rows[n]
 * to base+n and truncates. Returns 0, or -1 when rows is not an ascending path inside
 * the cache (nothing changes then). */
int bco_keep(float* cache, uint64_t width, uint64_t* len, uint64_t base,
             const uint32_t* rows, uint32_t nrows);

uint16_t bco_f32_to_f16(float x);
float bco_f16_to_f32(uint16_t h);
void bco_round_f16(float* x, size_t n); /* x[i] = f16(x[i]) as f32 */

/* splitmix64 state step and output. */
uint64_t bco_splitmix64(uint64_t* state);
/* n N(0,1) draws from seed: pairs by Box-Muller on two splitmix64 uniforms. */
void bco_normal(uint64_t seed, float* out, size_t n);

/* ---- The rest of the layer (bc_layer.c): TEST INFRASTRUCTURE as above. ----
 *   bcl_block, bcl_dequant_block  crates/bc-infer/src/quant.rs:69-82, 150-259
 *   bcl_scale_min_k4              crates/bc-infer/src/quant.rs:136-146
 *   bcl_ref_f32_to_f16            crates/bc-infer/src/quant.rs:114-131
 *   bcl_random_tensor             crates/bc-infer/src/fixtures.rs:66-92
 *   bcl_quantize_q8_0             crates/bc-infer/src/quant.rs:634-646
 *   bcl_matmul_f64                crates/bc-infer/src/gpu/mod.rs:193-196 (self_check's f64 sum)
 *   bcl_rms_norm                  crates/bc-infer/src/model.rs:381-388
 *   bcl_silu_mul, bcl_bias_add, bcl_add   model.rs:343, 371-377, 337
 * Pinned by tests/test_oracle.py against the reference's known-answer block tests
 * (quant.rs:650-729), hand-built blocks of every format and numpy restatements. */
/* ggml type numbers (quant.rs:35-49). */
#define BCL_F32 0u
#define BCL_F16 1u
#define BCL_Q4_0 2u
#define BCL_Q4_1 3u
#define BCL_Q5_0 6u
#define BCL_Q5_1 7u
#define BCL_Q8_0 8u
#define BCL_Q4K 12u
#define BCL_Q5K 13u
#define BCL_Q6K 14u
#define BCL_BF16 30u
int bcl_block(uint32_t ty, uint32_t* weights, uint32_t* bytes);
uint16_t bcl_ref_f32_to_f16(float x);
void bcl_scale_min_k4(uint32_t j, const uint8_t* q, float* sc, float* mn);
void bcl_dequant_block(uint32_t ty, const uint8_t* src, float* dst);
int bcl_dequant(uint32_t ty, const uint8_t* data, uint64_t rows, uint64_t cols, float* out);
int bcl_random_tensor(uint32_t ty, uint64_t rows, uint64_t cols, uint64_t seed, uint8_t* out);
void bcl_quantize_q8_0(const float* v, uint64_t n, uint8_t* out);
int bcl_matmul_f64(uint32_t ty, const uint8_t* data, uint64_t rows, uint64_t cols, const float* x, uint64_t n,
                   double* out);
void bcl_rms_norm(const float* x, const float* w, float* out, uint64_t rows, uint64_t cols, float eps);
void bcl_silu_mul(float* g, const float* u, uint64_t n);
void bcl_bias_add(float* x, const float* b, uint64_t n, uint64_t dim);
void bcl_add(float* x, const float* y, uint64_t n);

/* The sampler (bc_sample.c):
 *   bcs_argmax    crates/bc-infer/src/sample.rs:24-32
 *   bcs_uniform   crates/bc-infer/src/sample.rs:74-81 (splitmix64 one step, top 24 bits)
 *   bcs_sample    crates/bc-infer/src/sample.rs:35-71 (temperature, top-p nucleus, seeded draw)
 *   bcs_exp       f32::exp as the correctly rounded value (the reference leaves it to libm)
 * Pinned by the reference's greedy_and_nucleus test (sample.rs:78-89), the published
 * splitmix64 sequence, and properties with closed answers (tests/test_oracle_sample.py). */
uint32_t bcs_argmax(const float* s, uint32_t n);
float bcs_uniform(uint64_t seed);
float bcs_exp(float x);
uint32_t bcs_sample(const float* scores, uint32_t n, float temperature, float top_p, uint64_t seed,
                    uint64_t step);

#ifdef __cplusplus
}
#endif
#endif
