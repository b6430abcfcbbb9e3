/*
 * TEST INFRASTRUCTURE ONLY — the oracle.
 *
 * A CPU restatement of the MiniCPM-4 stack that tgtts-v4 runs on its GPU: the decode step
 * (crates/graph/src/decode.rs:456-736 with kernels/glsl/{norm,gemv,gemv_norm}.glsl and
 * {gemv_qkv_rope,attention_split,attention_combine,gemv_residual,gemv_gate_up,rmsnorm}.comp)
 * and the causal prefill (crates/graph/src/prefill.rs:218-413 with
 * {norm_rows,add_norm_rows,rope_rows,attention_rows,silu_mul_rows}.comp). The same source is
 * compiled twice: in double ("truth", the accuracy oracle) and in float (the fp32 CPU path the
 * benchmark times beside the GPU, standing in for burn's CPU model, which the reference tree
 * does not contain).
 *
 * Only tests/, the smoke check and the benchmark's CPU-baseline leg may load this library, and
 * only to hold results against (or as the CPU path timed beside the GPU). The GPU library never
 * links or calls it.
 *
 * Pinning (each function's checks live in tests/test_oracle.py):
 *   orc_rope_tables   — identity at t = 0, cos(1)/sin(1) at t = 1 for frequency 0
 *                       (decode.rs:1232-1242), and the f32 recipe against numpy float32.
 *   orc_rmsnorm       — testkit.safetensors:rms_layernorm KAT (fixtures/testkit.py:15-17),
 *                       closed form on random vectors, planted defect (gain left out).
 *   orc_attention     — brute-force softmax in numpy float64; one position returns v;
 *                       NaN past the position must not leak (crates/vulkan/tests/glsl.rs:617-699).
 *   orc_decode / orc_prefill — a whole stack against an independent torch float64 model built
 *                       from library ops (scaled_dot_product_attention, silu, matmul), prefill
 *                       against decode at every position, planted defects (positions shifted by
 *                       one, rotated residual LM) must fail the tolerance
 *                       (crates/graph/tests/decode.rs:252-255,372-378).
 */
#ifndef TGX_ORACLE_H
#define TGX_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* The shape a stack runs at (decode.rs:65-82). Weights are row-major float arrays, as upstream's
 * state_dict holds them after q/k/v and gate/up are joined along their outputs
 * (decode.rs:764-775). */
typedef struct {
    int hidden, inner, heads, kv_heads, head_dim, layers, capacity;
    double eps;
    int rope; /* whether q and k are rotated (decode.rs:47-50: the residual LM's are not) */
    const float* cos; /* [capacity][head_dim / 2], from orc_rope_tables */
    const float* sin;
} orc_shape;

typedef struct {
    const float* input_norm; /* [hidden] */
    const float* qkv;        /* [(heads + 2 kv_heads) head_dim][hidden]: q_proj; k_proj; v_proj */
    const float* o;          /* [hidden][heads head_dim] */
    const float* post_norm;  /* [hidden] */
    const float* gate_up;    /* [2 inner][hidden]: gate_proj; up_proj */
    const float* down;       /* [hidden][inner] */
} orc_layer;

/* LongRoPE's tables in f32, in the order Shape::rope_tables takes (decode.rs:146-168):
 * inv = 1 / theta^(2j/d), r = 1 / factor_j, angle = t * r * inv. factors may be NULL (all 1). */
void orc_rope_tables(int capacity, int head_dim, float theta, const double* factors, float* cos,
                     float* sin);

/* RMSNorm (kernels/glsl/norm.glsl:12-53): x * g / sqrt(mean(x^2) + eps). */
void orc_rmsnorm_f64(const double* x, const float* g, int k, double eps, double* out);
void orc_rmsnorm_f32(const float* x, const float* g, int k, float eps, float* out);

/* Softmax attention of `heads` query heads over positions 0..position of a
 * [kv_heads][capacity][head_dim] cache (attention_split.comp + attention_combine.comp).
 * Positions past `position` are never read. */
void orc_attention_f64(const double* q, const double* k_cache, const double* v_cache, int heads,
                       int kv_heads, int head_dim, int capacity, int position, double* out);

/* One decode step of one request: writes its keys and values at `position` of its cache
 * ([layers][kv_heads][capacity][head_dim] each), attends over 0..position, and returns the
 * hidden state after the final norm. Returns 0, or -1 for a position past the capacity. */
int orc_decode_f64(const orc_shape* s, const orc_layer* layers, const float* final_norm,
                   double* k_cache, double* v_cache, int position, const double* x, double* out);
int orc_decode_f32(const orc_shape* s, const orc_layer* layers, const float* final_norm,
                   float* k_cache, float* v_cache, int position, const float* x, float* out);

/* A causal run of `len` positions from `start` (Prefill::run, prefill.rs:473-503): the same
 * arithmetic as `len` decode steps, every position attending over the cache up to itself. */
int orc_prefill_f64(const orc_shape* s, const orc_layer* layers, const float* final_norm,
                    double* k_cache, double* v_cache, int start, int len, const double* x,
                    double* out);
int orc_prefill_f32(const orc_shape* s, const orc_layer* layers, const float* final_norm,
                    float* k_cache, float* v_cache, int start, int len, const float* x,
                    float* out);

/* Threads the fp32/fp64 paths use (OpenMP); 0 leaves the runtime's default. */
void orc_set_threads(int n);
int orc_threads(void);

#ifdef __cplusplus
}
#endif
#endif
