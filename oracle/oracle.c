/*
 * TEST INFRASTRUCTURE ONLY — the oracle (see oracle.h): the MiniCPM-4 stack on the CPU in double
 * and in float, from the same body (oracle_impl.h).
 */
#include "oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#define REAL double
#define SUFFIX f64
#define SQRT sqrt
#define EXP exp
#include "oracle_impl.h"
#undef REAL
#undef SUFFIX
#undef SQRT
#undef EXP

#define REAL float
#define SUFFIX f32
#define SQRT sqrtf
#define EXP expf
#include "oracle_impl.h"
#undef REAL
#undef SUFFIX
#undef SQRT
#undef EXP

void orc_rope_tables(int capacity, int head_dim, float theta, const double* factors, float* cos,
                     float* sin) {
    /* decode.rs:146-168: inv_freq in f32 from theta^(i / dim) for even i, divided by the factor
     * in f32; the angle t * r * inv in that f32 order. */
    int half = head_dim / 2;
    for (int t = 0; t < capacity; ++t) {
        for (int j = 0; j < half; ++j) {
            float inv = 1.0f / powf(theta, (float)(2 * j) / (float)head_dim);
            float r = 1.0f / (float)(factors ? factors[j] : 1.0);
            float f = (float)t * r * inv;
            cos[(size_t)t * half + j] = cosf(f);
            sin[(size_t)t * half + j] = sinf(f);
        }
    }
}

void orc_rmsnorm_f64(const double* x, const float* g, int k, double eps, double* out) {
    rmsnorm_in_f64(x, g, k, eps, out);
}

void orc_rmsnorm_f32(const float* x, const float* g, int k, float eps, float* out) {
    rmsnorm_in_f32(x, g, k, eps, out);
}

void orc_attention_f64(const double* q, const double* k_cache, const double* v_cache, int heads,
                       int kv_heads, int head_dim, int capacity, int position, double* out) {
    attend_f64(q, k_cache, v_cache, heads, kv_heads, head_dim, capacity, position, out);
}

int orc_decode_f64(const orc_shape* s, const orc_layer* layers, const float* final_norm,
                   double* k_cache, double* v_cache, int position, const double* x, double* out) {
    return step_f64(s, layers, final_norm, k_cache, v_cache, position, x, out);
}

int orc_decode_f32(const orc_shape* s, const orc_layer* layers, const float* final_norm,
                   float* k_cache, float* v_cache, int position, const float* x, float* out) {
    return step_f32(s, layers, final_norm, k_cache, v_cache, position, x, out);
}

int orc_prefill_f64(const orc_shape* s, const orc_layer* layers, const float* final_norm,
                    double* k_cache, double* v_cache, int start, int len, const double* x,
                    double* out) {
    if (start < 0 || len <= 0 || start + len > s->capacity) return -1;
    for (int i = 0; i < len; ++i) {
        int rc = step_f64(s, layers, final_norm, k_cache, v_cache, start + i,
                          x + (size_t)i * s->hidden, out + (size_t)i * s->hidden);
        if (rc) return rc;
    }
    return 0;
}

int orc_prefill_f32(const orc_shape* s, const orc_layer* layers, const float* final_norm,
                    float* k_cache, float* v_cache, int start, int len, const float* x,
                    float* out) {
    if (start < 0 || len <= 0 || start + len > s->capacity) return -1;
    for (int i = 0; i < len; ++i) {
        int rc = step_f32(s, layers, final_norm, k_cache, v_cache, start + i,
                          x + (size_t)i * s->hidden, out + (size_t)i * s->hidden);
        if (rc) return rc;
    }
    return 0;
}

void orc_set_threads(int n) {
#ifdef _OPENMP
    if (n > 0) omp_set_num_threads(n);
#else
    (void)n;
#endif
}

int orc_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}
