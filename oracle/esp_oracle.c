/*
 * esp_oracle.c — CPU restatement of esp's llama-family decoder forward in
 * f32 (TEST INFRASTRUCTURE: the parity checker and CPU baseline only).
 *
 * Op order follows the reference burn graph; reduction order inside a dot
 * product or a row sum is this file's own fixed order (16 interleaved
 * partial sums, then a pairwise fold), which burn-ndarray does not pin.
 * The reference's committed Transformers goldens pin the result to 2e-5.
 */
#include "esp_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#define LANES 16

static inline float bf16_to_f32(uint16_t b) {
    uint32_t u = (uint32_t)b << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}

static inline uint16_t f32_to_bf16_rne(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40); /* quiet NaN */
    uint32_t lsb = (u >> 16) & 1u;
    u += 0x7fffu + lsb;
    return (uint16_t)(u >> 16);
}

static inline float tget(orc_tensor t, size_t i) {
    if (t.dtype == ORC_BF16) return bf16_to_f32(((const uint16_t *)t.data)[i]);
    return ((const float *)t.data)[i];
}

static inline float fold16(float *acc) {
    for (int w = LANES / 2; w > 0; w /= 2)
        for (int j = 0; j < w; ++j) acc[j] += acc[j + w];
    return acc[0];
}

/* dot(x, row) over n with the fixed 16-lane order. */
static float dot_row(const float *x, orc_tensor w, size_t row, int n) {
    float acc[LANES] = {0};
    int j = 0;
    if (w.dtype == ORC_BF16) {
        const uint16_t *r = (const uint16_t *)w.data + row * (size_t)n;
        for (; j + LANES <= n; j += LANES)
            for (int l = 0; l < LANES; ++l) acc[l] += x[j + l] * bf16_to_f32(r[j + l]);
        for (; j < n; ++j) acc[j % LANES] += x[j] * bf16_to_f32(r[j]);
    } else {
        const float *r = (const float *)w.data + row * (size_t)n;
        for (; j + LANES <= n; j += LANES)
            for (int l = 0; l < LANES; ++l) acc[l] += x[j + l] * r[j + l];
        for (; j < n; ++j) acc[j % LANES] += x[j] * r[j];
    }
    return fold16(acc);
}

/* dot_row of one input row against four consecutive weight rows: the input
 * chunk is loaded once for all four; each dot keeps dot_row's own
 * accumulation order, so out[i] == dot_row(x, w, row + i, n) bit for bit. */
static void dot_row_w4(const float *x, orc_tensor w, size_t row, int n, float *out) {
    float acc[4][LANES] = {{0}};
    int j = 0;
    if (w.dtype == ORC_BF16) {
        const uint16_t *r = (const uint16_t *)w.data + row * (size_t)n;
        for (; j + LANES <= n; j += LANES)
            for (int i = 0; i < 4; ++i)
                for (int l = 0; l < LANES; ++l)
                    acc[i][l] += x[j + l] * bf16_to_f32(r[(size_t)i * n + j + l]);
    } else {
        const float *r = (const float *)w.data + row * (size_t)n;
        for (; j + LANES <= n; j += LANES)
            for (int i = 0; i < 4; ++i)
                for (int l = 0; l < LANES; ++l) acc[i][l] += x[j + l] * r[(size_t)i * n + j + l];
    }
    for (; j < n; ++j)
        for (int i = 0; i < 4; ++i) acc[i][j % LANES] += x[j] * tget(w, (row + i) * (size_t)n + j);
    for (int i = 0; i < 4; ++i) out[i] = fold16(acc[i]);
}

static float dot_f32(const float *a, const float *b, int n) {
    float acc[LANES] = {0};
    int j = 0;
    for (; j + LANES <= n; j += LANES)
        for (int l = 0; l < LANES; ++l) acc[l] += a[j + l] * b[j + l];
    for (; j < n; ++j) acc[j % LANES] += a[j] * b[j];
    return fold16(acc);
}

static float sumsq(const float *x, int n) { return dot_f32(x, x, n); }

/* Linear, dec/attention.rs:247-256 (burn Linear: x·W + b; W is HF [out,in]
 * here, so y[o] = dot(x, W[o]) + b[o]).  x [rows, in] -> y [rows, out]. */
static void linear(const float *x, int rows, int in_f, orc_tensor w, orc_tensor bias,
                   int out_f, float *y) {
    /* Rows go in blocks whose inputs fit a core's L2, outputs in fours
     * whose weight rows stay in L1 while the block's rows stream past; every
     * output is the same dot_row sum, so blocking does not change a bit. */
    int rb = (int)((512u * 1024u) / ((unsigned)in_f * sizeof(float)));
    if (rb < 1) rb = 1;
    for (int s0 = 0; s0 < rows; s0 += rb) {
        int s1 = s0 + rb < rows ? s0 + rb : rows;
#pragma omp parallel for schedule(static)
        for (int o4 = 0; o4 < (out_f + 3) / 4; ++o4) {
            int o = 4 * o4;
            if (o + 4 <= out_f) {
                for (int s = s0; s < s1; ++s) {
                    float v[4];
                    dot_row_w4(x + (size_t)s * in_f, w, (size_t)o, in_f, v);
                    for (int i = 0; i < 4; ++i) {
                        float b = bias.data ? tget(bias, (size_t)(o + i)) : 0.0f;
                        y[(size_t)s * out_f + o + i] = bias.data ? v[i] + b : v[i];
                    }
                }
                continue;
            }
            for (; o < out_f; ++o) {
                float b = bias.data ? tget(bias, (size_t)o) : 0.0f;
                for (int s = s0; s < s1; ++s) {
                    float v = dot_row(x + (size_t)s * in_f, w, (size_t)o, in_f);
                    y[(size_t)s * out_f + o] = bias.data ? v + b : v;
                }
            }
        }
    }
}

/* burn-nn RmsNorm as built at dec/layer.rs:27-33: y = x / sqrt(mean(x^2) + eps) * gamma. */
static void rmsnorm_row(const float *x, int n, orc_tensor gamma, float eps, float *y) {
    float mean = sumsq(x, n) / (float)n;
    float rms = sqrtf(mean + eps);
    for (int j = 0; j < n; ++j) y[j] = (x[j] / rms) * tget(gamma, (size_t)j);
}

static float silu(float x) { return x * (1.0f / (1.0f + expf(-x))); }
static float sigmoidf_(float x) { return 1.0f / (1.0f + expf(-x)); }

/* ---------------------------------------------------------------- RoPE */

/* dec/config.rs:158-180 RopeScaling::apply */
static float rope_scale(float freq, int scaling, float factor, float low, float high, int orig) {
    if (scaling == 1) return freq / factor;
    if (scaling == 2) {
        const float tau = 6.28318530717958647692f; /* std::f32::consts::TAU */
        float wavelength = tau / freq;
        float original = (float)orig;
        if (wavelength < original / high) return freq;
        if (wavelength > original / low) return freq / factor;
        float smooth = (original / wavelength - low) / (high - low);
        return (1.0f - smooth) * freq / factor + smooth * freq;
    }
    return freq;
}

/* dec/attention.rs:58-95 LlamaRotaryEncoding::with_scaling */
void orc_rope_table(int max_pos, int head_dim, float theta, int scaling, float factor,
                    float low_freq, float high_freq, int orig_max, float *cos_out,
                    float *sin_out) {
    int half = head_dim / 2;
    for (int p = 0; p < max_pos; ++p) {
        for (int i = 0; i < half; ++i) {
            float inv = 1.0f / powf(theta, (float)(2 * i) / (float)head_dim);
            inv = rope_scale(inv, scaling, factor, low_freq, high_freq, orig_max);
            float angle = (float)p * inv;
            float c = cosf(angle), s = sinf(angle);
            cos_out[(size_t)p * head_dim + i] = c;
            cos_out[(size_t)p * head_dim + half + i] = c;
            sin_out[(size_t)p * head_dim + i] = s;
            sin_out[(size_t)p * head_dim + half + i] = s;
        }
    }
}

/* dec/attention.rs:99-123 apply: x*cos + cat(-x2, x1)*sin at absolute pos. */
static void rope_apply(float *x, int hd, const float *cos_row, const float *sin_row) {
    int half = hd / 2;
    float tmp[1024];
    float *r = hd <= 1024 ? tmp : (float *)malloc(sizeof(float) * (size_t)hd);
    for (int j = 0; j < hd; ++j) {
        float rot = j < half ? -x[j + half] : x[j - half];
        r[j] = x[j] * cos_row[j] + rot * sin_row[j];
    }
    memcpy(x, r, sizeof(float) * (size_t)hd);
    if (r != tmp) free(r);
}

/* ---------------------------------------------------------------- KV */

struct orc_kv {
    int layers, n_kv, hd, max_ctx, position;
    float *k, *v; /* [layers][n_kv][max_ctx][hd] */
};

orc_kv *orc_kv_create(const orc_model *m, int max_ctx) {
    orc_kv *kv = (orc_kv *)calloc(1, sizeof(orc_kv));
    if (!kv) return NULL;
    kv->layers = m->layers;
    kv->n_kv = m->n_kv_heads;
    kv->hd = m->head_dim;
    kv->max_ctx = max_ctx;
    size_t n = (size_t)m->layers * m->n_kv_heads * (size_t)max_ctx * m->head_dim;
    kv->k = (float *)calloc(n, sizeof(float));
    kv->v = (float *)calloc(n, sizeof(float));
    if (!kv->k || !kv->v) {
        orc_kv_destroy(kv);
        return NULL;
    }
    return kv;
}

void orc_kv_destroy(orc_kv *kv) {
    if (!kv) return;
    free(kv->k);
    free(kv->v);
    free(kv);
}

int orc_kv_position(const orc_kv *kv) { return kv->position; }

static inline float *kv_row(const orc_kv *kv, float *base, int l, int h, int t) {
    return base + (((size_t)l * kv->n_kv + h) * (size_t)kv->max_ctx + t) * kv->hd;
}

/* ---------------------------------------------------------------- MLP */

/* moe.rs:76-90 SwiGLU MLP (Expert::forward = down(silu(x·gate) * (x·up)))
 * over rows, parallel over output features. */
static void dense_mlp(const float *x, int rows, int h, int f, orc_tensor gate, orc_tensor up,
                      orc_tensor down, float *act, float *y) {
    /* row blocks as in linear() */
    int rb = (int)((512u * 1024u) / ((unsigned)h * sizeof(float)));
    if (rb < 1) rb = 1;
    for (int s0 = 0; s0 < rows; s0 += rb) {
        int s1 = s0 + rb < rows ? s0 + rb : rows;
#pragma omp parallel for schedule(static)
        for (int j4 = 0; j4 < (f + 3) / 4; ++j4) {
            int j = 4 * j4;
            if (j + 4 <= f) {
                for (int s = s0; s < s1; ++s) {
                    float g[4], u[4];
                    dot_row_w4(x + (size_t)s * h, gate, (size_t)j, h, g);
                    dot_row_w4(x + (size_t)s * h, up, (size_t)j, h, u);
                    for (int i = 0; i < 4; ++i) act[(size_t)s * f + j + i] = silu(g[i]) * u[i];
                }
                continue;
            }
            for (; j < f; ++j) {
                for (int s = s0; s < s1; ++s) {
                    const float *xr = x + (size_t)s * h;
                    float g = dot_row(xr, gate, (size_t)j, h);
                    float u = dot_row(xr, up, (size_t)j, h);
                    act[(size_t)s * f + j] = silu(g) * u;
                }
            }
        }
    }
    orc_tensor none = {0};
    linear(act, rows, f, down, none, h, y);
}

/* moe.rs:135-256 DecoderMlp::forward (Moe arm). Returns 0 or -2/-3.
 * Routing per row first; then, as the reference does, expert by expert in
 * ascending id over the rows that chose it (moe.rs:183-251), each row
 * adding delta * weight in that order; then the shared expert. */
static int moe_mlp(const orc_model *m, int l, const float *x, int rows, float *y) {
    const orc_tensor *lt = m->layer + (size_t)l * ORC_LAYER_SLOTS;
    int h = m->hidden, e_n = m->n_experts, k = m->top_k;
    int f = m->moe_ffn, fs = m->shared_ffn;
    int status = 0;
    float *probs = (float *)malloc(sizeof(float) * (size_t)rows * e_n);
    float *wsel = (float *)calloc((size_t)rows * e_n, sizeof(float));
    unsigned char *chosen = (unsigned char *)calloc((size_t)rows * e_n, 1);
    orc_tensor none = {0};
    linear(x, rows, h, lt[ORC_ROUTER], none, e_n, probs);
#pragma omp parallel
    {
        int *order = (int *)malloc(sizeof(int) * (size_t)e_n);
#pragma omp for schedule(static)
        for (int s = 0; s < rows; ++s) {
            float *p = probs + (size_t)s * e_n;
            float *yr = y + (size_t)s * h;
            for (int j = 0; j < h; ++j) yr[j] = 0.0f;
            /* fp32 softmax over all experts (moe.rs:156-159) */
            float mx = -INFINITY;
            for (int e = 0; e < e_n; ++e) mx = fmaxf(mx, p[e]);
            float sum = 0.0f;
            for (int e = 0; e < e_n; ++e) {
                p[e] = expf(p[e] - mx);
                sum += p[e];
            }
            int bad = 0;
            for (int e = 0; e < e_n; ++e) {
                p[e] = p[e] / sum;
                if (!isfinite(p[e])) bad = 1;
            }
            if (bad) {
#pragma omp atomic write
                status = -2;
                continue;
            }
            /* sort by probability desc, then id asc (moe.rs:166) */
            for (int e = 0; e < e_n; ++e) order[e] = e;
            for (int a = 1; a < e_n; ++a) {
                int v = order[a], b = a - 1;
                while (b >= 0 && (p[order[b]] < p[v] || (p[order[b]] == p[v] && order[b] > v))) {
                    order[b + 1] = order[b];
                    --b;
                }
                order[b + 1] = v;
            }
            float mass = 1.0f;
            if (m->norm_topk) {
                mass = 0.0f;
                for (int i = 0; i < k; ++i) mass += p[order[i]];
            }
            if (!isfinite(mass) || mass <= 0.0f) {
#pragma omp atomic write
                status = -3;
                continue;
            }
            for (int i = 0; i < k; ++i) {
                chosen[(size_t)s * e_n + order[i]] = 1;
                wsel[(size_t)s * e_n + order[i]] = p[order[i]] / mass;
            }
        }
        free(order);
    }
    int fmax = f > fs ? f : fs;
    int *idx = (int *)malloc(sizeof(int) * (size_t)(rows > 0 ? rows : 1));
    float *xs = (float *)malloc(sizeof(float) * (size_t)rows * h);
    float *ys = (float *)malloc(sizeof(float) * (size_t)rows * h);
    float *act = (float *)malloc(sizeof(float) * (size_t)rows * (size_t)(fmax > 0 ? fmax : 1));
    /* experts in ascending id, each row adding delta*w (moe.rs:183-245) */
    for (int e = 0; e < e_n && status == 0; ++e) {
        int ne = 0;
        for (int s = 0; s < rows; ++s)
            if (chosen[(size_t)s * e_n + e]) idx[ne++] = s;
        if (ne == 0) continue;
        for (int i = 0; i < ne; ++i)
            memcpy(xs + (size_t)i * h, x + (size_t)idx[i] * h, sizeof(float) * h);
        const orc_tensor *ex = m->experts + ((size_t)l * e_n + e) * 3;
        dense_mlp(xs, ne, h, f, ex[0], ex[1], ex[2], act, ys);
#pragma omp parallel for schedule(static)
        for (int i = 0; i < ne; ++i) {
            float w = wsel[(size_t)idx[i] * e_n + e];
            float *yr = y + (size_t)idx[i] * h;
            const float *d = ys + (size_t)i * h;
            for (int j = 0; j < h; ++j) yr[j] = yr[j] + d[j] * w;
        }
    }
    /* + sigmoid(shared_gate·x) * shared(x) (moe.rs:253) */
    if (status == 0 && fs > 0 && lt[ORC_SH_GATE].data) {
        dense_mlp(x, rows, h, fs, lt[ORC_SH_GATE], lt[ORC_SH_UP], lt[ORC_SH_DOWN], act, ys);
#pragma omp parallel for schedule(static)
        for (int s = 0; s < rows; ++s) {
            float g = sigmoidf_(dot_row(x + (size_t)s * h, lt[ORC_SHARED_GATE], 0, h));
            float *yr = y + (size_t)s * h;
            const float *d = ys + (size_t)s * h;
            for (int j = 0; j < h; ++j) yr[j] = yr[j] + g * d[j];
        }
    }
    free(idx);
    free(xs);
    free(ys);
    free(act);
    free(probs);
    free(wsel);
    free(chosen);
    return status;
}

/* ---------------------------------------------------------------- forward */

/* model.rs:502-666 + layer.rs:115-153 + attention.rs:292-404 */
int orc_forward_last(const orc_model *m, orc_kv *kv, const int32_t *ids, int n, float *logits_out,
                     float *all_logits) {
    int start = kv->position;
    if (n <= 0 || start + n > m->max_pos || start + n > kv->max_ctx) return -1;
    for (int s = 0; s < n; ++s)
        if (ids[s] < 0 || ids[s] >= m->vocab) return -1;
    int H = m->hidden, nq = m->n_heads, nkv = m->n_kv_heads, hd = m->head_dim;
    int qw = nq * hd, kvw = nkv * hd, group = nq / nkv;
    int fmax = m->ffn;
    if (m->moe_ffn > fmax) fmax = m->moe_ffn;
    if (m->shared_ffn > fmax) fmax = m->shared_ffn;
    size_t rows = (size_t)n;
    float *h = (float *)malloc(sizeof(float) * rows * H);
    float *xn = (float *)malloc(sizeof(float) * rows * H);
    float *q = (float *)malloc(sizeof(float) * rows * qw);
    float *kk = (float *)malloc(sizeof(float) * rows * kvw);
    float *vv = (float *)malloc(sizeof(float) * rows * kvw);
    float *att = (float *)malloc(sizeof(float) * rows * qw);
    float *tmp = (float *)malloc(sizeof(float) * rows * H);
    float *act = (float *)malloc(sizeof(float) * rows * (size_t)(fmax > 0 ? fmax : 1));
    if (!h || !xn || !q || !kk || !vv || !att || !tmp || !act) {
        free(h); free(xn); free(q); free(kk); free(vv); free(att); free(tmp); free(act);
        return -4;
    }
    int status = 0;
    float inv_sqrt = sqrtf((float)hd);

    /* TokenEmbedding::forward (model.rs:59-62) */
    for (int s = 0; s < n; ++s)
        for (int j = 0; j < H; ++j) h[(size_t)s * H + j] = tget(m->embed, (size_t)ids[s] * H + j);

    for (int l = 0; l < m->layers && status == 0; ++l) {
        const orc_tensor *lt = m->layer + (size_t)l * ORC_LAYER_SLOTS;
        /* input RMSNorm (layer.rs:125) */
        for (int s = 0; s < n; ++s)
            rmsnorm_row(h + (size_t)s * H, H, lt[ORC_IN_NORM], m->rms_eps, xn + (size_t)s * H);
        /* q/k/v projections (attention.rs:309-311) */
        orc_tensor none = {0};
        linear(xn, n, H, lt[ORC_Q], m->qkv_bias ? lt[ORC_Q_BIAS] : none, qw, q);
        linear(xn, n, H, lt[ORC_K], m->qkv_bias ? lt[ORC_K_BIAS] : none, kvw, kk);
        linear(xn, n, H, lt[ORC_V], m->qkv_bias ? lt[ORC_V_BIAS] : none, kvw, vv);
        /* QK norm (attention.rs:312-319), then RoPE (attention.rs:323-324) */
        for (int s = 0; s < n; ++s) {
            const float *c = m->rope_cos + (size_t)(start + s) * hd;
            const float *sn = m->rope_sin + (size_t)(start + s) * hd;
            for (int hh = 0; hh < nq; ++hh) {
                float *x = q + (size_t)s * qw + (size_t)hh * hd;
                if (m->qk_norm) rmsnorm_row(x, hd, lt[ORC_Q_NORM], m->rms_eps, x);
                rope_apply(x, hd, c, sn);
            }
            for (int hh = 0; hh < nkv; ++hh) {
                float *x = kk + (size_t)s * kvw + (size_t)hh * hd;
                if (m->qk_norm) rmsnorm_row(x, hd, lt[ORC_K_NORM], m->rms_eps, x);
                rope_apply(x, hd, c, sn);
                /* LayerKvCache::append (attention.rs:136-148) */
                memcpy(kv_row(kv, kv->k, l, hh, start + s), x, sizeof(float) * hd);
                memcpy(kv_row(kv, kv->v, l, hh, start + s), vv + (size_t)s * kvw + (size_t)hh * hd,
                       sizeof(float) * hd);
            }
        }
        int total = start + n;
        int window = m->layer_window ? m->layer_window[l] : 0;
        /* scores / sqrt(hd), mask, softmax, ·V (attention.rs:345-397) */
#pragma omp parallel
        {
            float *sc = (float *)malloc(sizeof(float) * (size_t)total);
#pragma omp for collapse(2) schedule(static)
            for (int s = 0; s < n; ++s) {
                for (int hh = 0; hh < nq; ++hh) {
                    int kvh = hh / group;
                    int qpos = start + s;
                    const float *qr = q + (size_t)s * qw + (size_t)hh * hd;
                    float mx = -INFINITY;
                    for (int t = 0; t < total; ++t) {
                        int masked = t > qpos ||
                                     (window > 0 && qpos - (t < qpos ? t : qpos) >= window);
                        if (masked) {
                            sc[t] = -INFINITY;
                        } else {
                            sc[t] = dot_f32(qr, kv_row(kv, kv->k, l, kvh, t), hd) / inv_sqrt;
                        }
                        mx = fmaxf(mx, sc[t]);
                    }
                    float sum = 0.0f;
                    for (int t = 0; t < total; ++t) {
                        sc[t] = expf(sc[t] - mx);
                        sum += sc[t];
                    }
                    float *o = att + (size_t)s * qw + (size_t)hh * hd;
                    for (int j = 0; j < hd; ++j) o[j] = 0.0f;
                    for (int t = 0; t < total; ++t) {
                        float p = sc[t] / sum;
                        if (p == 0.0f) continue;
                        const float *vr = kv_row(kv, kv->v, l, kvh, t);
                        for (int j = 0; j < hd; ++j) o[j] += p * vr[j];
                    }
                }
            }
            free(sc);
        }
        /* o_proj (attention.rs:403) + residual (layer.rs:123-131) */
        linear(att, n, qw, lt[ORC_O], m->o_bias ? lt[ORC_O_BIAS] : none, H, tmp);
        for (size_t i = 0; i < rows * H; ++i) h[i] = h[i] + tmp[i];
        /* post-attention RMSNorm + MLP + residual (layer.rs:147-151) */
        for (int s = 0; s < n; ++s)
            rmsnorm_row(h + (size_t)s * H, H, lt[ORC_POST_NORM], m->rms_eps, xn + (size_t)s * H);
        if (m->layer_is_moe && m->layer_is_moe[l]) {
            status = moe_mlp(m, l, xn, n, tmp);
        } else {
            dense_mlp(xn, n, H, m->ffn, lt[ORC_GATE], lt[ORC_UP], lt[ORC_DOWN], act, tmp);
        }
        for (size_t i = 0; i < rows * H; ++i) h[i] = h[i] + tmp[i];
    }
    if (status == 0) {
        kv->position = start + n;
        /* final RmsNorm (model.rs:661-665) then the head on the last row
         * (model.rs:531-538); tied head = embedding rows (model.rs:167-169). */
        orc_tensor head = m->lm_head.data ? m->lm_head : m->embed;
        int first = all_logits ? 0 : n - 1;
        for (int s = first; s < n; ++s)
            rmsnorm_row(h + (size_t)s * H, H, m->final_norm, m->rms_eps, xn + (size_t)s * H);
        orc_tensor none = {0};
        if (all_logits) linear(xn, n, H, head, none, m->vocab, all_logits);
        if (logits_out) linear(xn + (size_t)(n - 1) * H, 1, H, head, none, m->vocab, logits_out);
    }
    free(h); free(xn); free(q); free(kk); free(vv); free(att); free(tmp); free(act);
    return status;
}

/* ---------------------------------------------------------------- LoRA */

/* lora.rs:93-97 add_delta: base + (A^T B^T) * scale, here in HF [out,in]. */
void orc_lora_merge(orc_tensor base, const float *a, const float *b, int out_f, int in_f, int rank,
                    float scale, float *merged) {
#pragma omp parallel for schedule(static)
    for (int o = 0; o < out_f; ++o) {
        for (int i = 0; i < in_f; ++i) {
            float d = 0.0f;
            for (int r = 0; r < rank; ++r) d += a[(size_t)r * in_f + i] * b[(size_t)o * rank + r];
            merged[(size_t)o * in_f + i] = tget(base, (size_t)o * in_f + i) + d * scale;
        }
    }
}

/* ---------------------------------------------------------------- picking */

/* lowest id wins among equal maxima (provider.rs:808-815); NaN rows are
 * masked before this in the constrained path. */
int32_t orc_argmax(const float *row, int n) {
    int32_t best = 0;
    for (int i = 1; i < n; ++i)
        if (row[i] > row[best] || (isnan(row[i]) && !isnan(row[best]))) best = i;
    return best;
}

/* constraint.rs:277-297 */
int orc_mask(float *row, int n, const uint32_t *allowed_bits) {
    int any = 0;
    for (int i = 0; i < n; ++i) {
        int allowed = (allowed_bits[i >> 5] >> (i & 31)) & 1u;
        if (!allowed || !isfinite(row[i])) row[i] = -INFINITY;
        else ++any;
    }
    return any;
}

/* sample.rs:38-45 */
uint64_t orc_splitmix64_next(uint64_t *state) {
    *state += 0x9E3779B97F4A7C15ull;
    uint64_t z = *state;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

/* sample.rs:64-69 */
uint64_t orc_skip_draws(uint64_t state, uint64_t draws) {
    return state + 0x9E3779B97F4A7C15ull * draws;
}

/* f32::total_cmp key: larger key = later in ascending total order. */
static inline int64_t total_key(float f) {
    int32_t i;
    memcpy(&i, &f, 4);
    i ^= (int32_t)(((uint32_t)(i >> 31)) >> 1);
    return (int64_t)i;
}

typedef struct {
    float w;
    int32_t id;
} wid;

static int cmp_desc(const void *pa, const void *pb) {
    const wid *a = (const wid *)pa, *b = (const wid *)pb;
    int64_t ka = total_key(a->w), kb = total_key(b->w);
    if (ka != kb) return ka > kb ? -1 : 1;
    return a->id < b->id ? -1 : (a->id > b->id);
}

/* sample.rs:83-121 Sampler::sample */
int32_t orc_sample(const float *row, int n, float temperature, float top_p, uint64_t *state) {
    float inv_t = 1.0f / temperature;
    float mx = -INFINITY;
    for (int i = 0; i < n; ++i) mx = fmaxf(mx, row[i]);
    wid *w = (wid *)malloc(sizeof(wid) * (size_t)n);
    for (int i = 0; i < n; ++i) {
        w[i].w = expf((row[i] - mx) * inv_t);
        w[i].id = i;
    }
    qsort(w, (size_t)n, sizeof(wid), cmp_desc);
    int keep = n;
    if (top_p >= 0.0f) {
        float total = -0.0f;
        for (int i = 0; i < n; ++i) total += w[i].w;
        float p = top_p < 0.0f ? 0.0f : (top_p > 1.0f ? 1.0f : top_p);
        float target = total * p;
        float mass = 0.0f;
        keep = 0;
        for (int i = 0; i < n; ++i) {
            mass += w[i].w;
            keep = i + 1;
            if (mass >= target) break;
        }
        if (keep < 1) keep = 1;
    }
    float total = -0.0f;
    for (int i = 0; i < keep; ++i) total += w[i].w;
    uint64_t x = orc_splitmix64_next(state);
    float u = (float)((double)(x >> 11) / 9007199254740992.0) * total;
    int32_t out = keep > 0 ? w[keep - 1].id : 0;
    for (int i = 0; i < keep; ++i) {
        u -= w[i].w;
        if (u <= 0.0f) {
            out = w[i].id;
            break;
        }
    }
    free(w);
    return out;
}

/* ---------------------------------------------------------------- inputs */

void orc_fill_normal(uint64_t seed, size_t n, float std, int dtype, void *out) {
#pragma omp parallel for schedule(static)
    for (size_t p = 0; p < (n + 1) / 2; ++p) {
        uint64_t st = seed + 0x9E3779B97F4A7C15ull * (uint64_t)(2 * p);
        uint64_t x1 = orc_splitmix64_next(&st);
        uint64_t x2 = orc_splitmix64_next(&st);
        double u1 = ((double)(x1 >> 11) + 1.0) / 9007199254740992.0;
        double u2 = (double)(x2 >> 11) / 9007199254740992.0;
        double r = sqrt(-2.0 * log(u1));
        double t = 6.283185307179586476925 * u2;
        float v[2] = {(float)(r * cos(t) * std), (float)(r * sin(t) * std)};
        for (int j = 0; j < 2; ++j) {
            size_t i = 2 * p + j;
            if (i >= n) break;
            if (dtype == ORC_BF16) ((uint16_t *)out)[i] = f32_to_bf16_rne(v[j]);
            else ((float *)out)[i] = v[j];
        }
    }
}

void orc_kv_fill_synthetic(orc_kv *kv, int position, uint64_t seed) {
    size_t n = (size_t)kv->layers * kv->n_kv * (size_t)kv->max_ctx * kv->hd;
    orc_fill_normal(seed, n, 1.0f, ORC_F32, kv->k);
    orc_fill_normal(seed ^ 0x5bd1e995u, n, 1.0f, ORC_F32, kv->v);
    kv->position = position;
}

void orc_set_threads(int n) {
#ifdef _OPENMP
    omp_set_num_threads(n);
#else
    (void)n;
#endif
}

int orc_get_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}
