/*
 * TEST INFRASTRUCTURE ONLY — the body of the oracle, included by oracle.c once with REAL = double
 * (suffix f64) and once with REAL = float (suffix f32). See oracle.h for what it restates.
 */
#define CAT2(a, b) a##_##b
#define CAT(a, b) CAT2(a, b)
#define FN(name) CAT(name, SUFFIX)

/* y[r] = sum_k W[r][k] x[k] for rows [0, rows), accumulated in REAL in k order.
 * The GEMVs of kernels/glsl/gemv.glsl:82-127 (f32 sums of f16 products). */
static void FN(gemv)(const float* w, const REAL* x, int rows, int k, REAL* y) {
#pragma omp parallel for schedule(static)
    for (int r = 0; r < rows; ++r) {
        const float* row = w + (size_t)r * k;
        REAL acc = 0;
        for (int i = 0; i < k; ++i) acc += (REAL)row[i] * x[i];
        y[r] = acc;
    }
}

/* RMSNorm as upstream's MiniCPMRMSNorm (kernels/glsl/norm.glsl:12-29, :47-53). */
static void FN(rmsnorm_in)(const REAL* x, const float* g, int k, REAL eps, REAL* out) {
    REAL squares = 0;
    for (int i = 0; i < k; ++i) squares += x[i] * x[i];
    REAL scale = (REAL)1 / SQRT(squares / (REAL)k + eps);
    for (int i = 0; i < k; ++i) out[i] = x[i] * scale * (REAL)g[i];
}

/* Rotate-half RoPE of one head at `pos` (gemv_qkv_rope.comp:86-94): the pairs (i, i + d/2),
 * a' = a cos - c sin, c' = c cos + a sin, with the host's f32 tables. */
static void FN(rope_head)(REAL* v, int head_dim, const float* cos, const float* sin, int pos) {
    int half = head_dim / 2;
    for (int i = 0; i < half; ++i) {
        REAL co = (REAL)cos[(size_t)pos * half + i];
        REAL si = (REAL)sin[(size_t)pos * half + i];
        REAL a = v[i], c = v[i + half];
        v[i] = a * co - c * si;
        v[i + half] = c * co + a * si;
    }
}

/* Softmax attention over 0..position (attention_split.comp:52-111, attention_combine.comp:29-57):
 * scores q.k / sqrt(d), max-subtracted exponentials, weighted sum of v, divided by the total. */
static void FN(attend)(const REAL* q, const REAL* kc, const REAL* vc, int heads, int kv_heads,
                       int head_dim, int capacity, int position, REAL* out) {
    int group = heads / kv_heads;
    REAL scale = (REAL)1 / SQRT((REAL)head_dim);
#pragma omp parallel for schedule(static)
    for (int h = 0; h < heads; ++h) {
        int kv = h / group;
        const REAL* qh = q + (size_t)h * head_dim;
        const REAL* kbase = kc + (size_t)kv * capacity * head_dim;
        const REAL* vbase = vc + (size_t)kv * capacity * head_dim;
        REAL* o = out + (size_t)h * head_dim;
        REAL m = -INFINITY;
        REAL* scores = (REAL*)malloc(sizeof(REAL) * (size_t)(position + 1));
        for (int p = 0; p <= position; ++p) {
            const REAL* kp = kbase + (size_t)p * head_dim;
            REAL s = 0;
            for (int d = 0; d < head_dim; ++d) s += qh[d] * kp[d];
            s *= scale;
            scores[p] = s;
            if (s > m) m = s;
        }
        REAL total = 0;
        for (int d = 0; d < head_dim; ++d) o[d] = 0;
        for (int p = 0; p <= position; ++p) {
            REAL e = EXP(scores[p] - m);
            total += e;
            const REAL* vp = vbase + (size_t)p * head_dim;
            for (int d = 0; d < head_dim; ++d) o[d] += e * vp[d];
        }
        for (int d = 0; d < head_dim; ++d) o[d] /= total;
        free(scores);
    }
}

/* One position through every layer (decode_batch_graph's op order, decode.rs:630-723):
 * qkv_rope, attention, o_proj + residual, norm + gate_up + SiLU, down_proj + residual; then the
 * final norm. */
static int FN(step)(const orc_shape* s, const orc_layer* layers, const float* final_norm,
                    REAL* k_cache, REAL* v_cache, int position, const REAL* x, REAL* out) {
    if (position < 0 || position >= s->capacity) return -1;
    const int h = s->hidden, d = s->head_dim, H = s->heads, KV = s->kv_heads, I = s->inner;
    const int qkv_rows = (H + 2 * KV) * d;
    const REAL eps = (REAL)s->eps;
    REAL* hs = (REAL*)malloc(sizeof(REAL) * h);
    REAL* normed = (REAL*)malloc(sizeof(REAL) * h);
    REAL* qkv = (REAL*)malloc(sizeof(REAL) * qkv_rows);
    REAL* att = (REAL*)malloc(sizeof(REAL) * H * d);
    REAL* o = (REAL*)malloc(sizeof(REAL) * h);
    REAL* gu = (REAL*)malloc(sizeof(REAL) * 2 * I);
    REAL* mlp = (REAL*)malloc(sizeof(REAL) * I);
    memcpy(hs, x, sizeof(REAL) * h);
    const size_t layer_cache = (size_t)KV * s->capacity * d;
    for (int l = 0; l < s->layers; ++l) {
        const orc_layer* w = &layers[l];
        REAL* kc = k_cache + (size_t)l * layer_cache;
        REAL* vc = v_cache + (size_t)l * layer_cache;
        FN(rmsnorm_in)(hs, w->input_norm, h, eps, normed);
        FN(gemv)(w->qkv, normed, qkv_rows, h, qkv);
        for (int head = 0; head < H + KV; ++head) {
            if (s->rope) FN(rope_head)(qkv + (size_t)head * d, d, s->cos, s->sin, position);
        }
        for (int kv = 0; kv < KV; ++kv) {
            memcpy(kc + ((size_t)kv * s->capacity + position) * d, qkv + (size_t)(H + kv) * d,
                   sizeof(REAL) * d);
            memcpy(vc + ((size_t)kv * s->capacity + position) * d,
                   qkv + (size_t)(H + KV + kv) * d, sizeof(REAL) * d);
        }
        FN(attend)(qkv, kc, vc, H, KV, d, s->capacity, position, att);
        FN(gemv)(w->o, att, h, H * d, o);
        for (int i = 0; i < h; ++i) hs[i] += o[i];
        FN(rmsnorm_in)(hs, w->post_norm, h, eps, normed);
        FN(gemv)(w->gate_up, normed, 2 * I, h, gu);
        for (int i = 0; i < I; ++i) {
            REAL gate = gu[i], up = gu[I + i];
            mlp[i] = gate / ((REAL)1 + EXP(-gate)) * up;
        }
        FN(gemv)(w->down, mlp, h, I, o);
        for (int i = 0; i < h; ++i) hs[i] += o[i];
    }
    FN(rmsnorm_in)(hs, final_norm, h, eps, out);
    free(hs); free(normed); free(qkv); free(att); free(o); free(gu); free(mlp);
    return 0;
}

#undef FN
#undef CAT
#undef CAT2
