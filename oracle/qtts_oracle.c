/*
 * qtts_oracle.c — CPU restatement of the reference's per-code loop.
 *
 * TEST INFRASTRUCTURE ONLY (what the parity tests compare with, and the
 * timed CPU baseline);
 * the product library never links or calls it.  Every function cites the
 * reference lines whose arithmetic order it follows.  Compile with
 * -O3 -ffp-contract=off and no -march flag (Cargo.toml:20-23 release profile,
 * default x86-64 target): no FMA contraction and no reassociation, so each
 * f32 operation rounds where the Rust code rounds.
 */
#define _GNU_SOURCE
#include "qtts_oracle.h"

#include <math.h>
#include <pthread.h>
#include <sched.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#define Q4_GROUP 32 /* Q4_GROUP_SIZE, src/gemv.rs:18 */

/* ------------------------------------------------------------------------ */
/* helpers                                                                   */
/* ------------------------------------------------------------------------ */

/* half::f16::to_f32 (half 2.7.1): exact widening, subnormals included. */
float qor_f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t ex = (h >> 10) & 0x1Fu;
    uint32_t man = h & 0x3FFu;
    uint32_t bits;
    float f;
    if (ex == 0) {
        f = (float)man * 0x1p-24f; /* exact: man < 2^10 */
        memcpy(&bits, &f, 4);
        bits |= sign;
    } else if (ex == 31) {
        bits = sign | 0x7F800000u | (man << 13);
    } else {
        bits = sign | ((ex + 112u) << 23) | (man << 13);
    }
    memcpy(&f, &bits, 4);
    return f;
}

int32_t qor_available_parallelism(void) {
    cpu_set_t set;
    int n = 0;
    if (sched_getaffinity(0, sizeof(set), &set) == 0) n = CPU_COUNT(&set);
    if (n <= 0) n = 6; /* unwrap_or(6), src/gemv.rs:269 */
    /* cgroup v2 quota ("max" or "<quota> <period>"), as std does on Linux. */
    FILE *f = fopen("/sys/fs/cgroup/cpu.max", "r");
    if (f) {
        char q[64];
        long period = 0;
        if (fscanf(f, "%63s %ld", q, &period) == 2 && strcmp(q, "max") != 0 && period > 0) {
            long quota = atol(q);
            long lim = quota / period;
            if (lim < 1) lim = 1;
            if (lim < n) n = (int)lim;
        }
        fclose(f);
    }
    return n;
}

static void *xcalloc(size_t n, size_t sz) {
    void *p = calloc(n ? n : 1, sz ? sz : 1);
    if (!p) {
        fprintf(stderr, "oracle: out of memory\n");
        abort();
    }
    return p;
}

/* ------------------------------------------------------------------------ */
/* Q4 GEMV: gemv_q4_inner, src/gemv.rs:222-261                               */
/* ------------------------------------------------------------------------ */
static void gemv_q4_inner(const float *input, const uint8_t *packed, const uint16_t *scales, int32_t n,
                          int32_t k_start, int32_t k_end, float *output /* [n], zeroed */) {
    const int32_t groups_per_row = n / Q4_GROUP;
    const int32_t packed_per_group = Q4_GROUP / 2;
    const size_t packed_per_row = (size_t)groups_per_row * packed_per_group;
    for (int32_t ki = k_start; ki < k_end; ki++) {
        const float input_val = input[ki];
        if (input_val == 0.0f) continue;
        const size_t scale_base = (size_t)ki * groups_per_row;
        const size_t pack_base = (size_t)ki * packed_per_row;
        for (int32_t g = 0; g < groups_per_row; g++) {
            const float s = qor_f16_to_f32(scales[scale_base + g]) * input_val;
            if (s == 0.0f) continue;
            const float lut[16] = {s * -8.0f, s * -7.0f, s * -6.0f, s * -5.0f, s * -4.0f, s * -3.0f,
                                   s * -2.0f, s * -1.0f, 0.0f,       s,          s * 2.0f,  s * 3.0f,
                                   s * 4.0f,  s * 5.0f,  s * 6.0f,  s * 7.0f};
            const uint8_t *p = packed + pack_base + (size_t)g * packed_per_group;
            float *o = output + (size_t)g * Q4_GROUP;
            for (int32_t j = 0; j < packed_per_group; j++) {
                const uint8_t byte = p[j];
                o[j * 2] += lut[byte & 0x0F];
                o[j * 2 + 1] += lut[byte >> 4];
            }
        }
    }
}

typedef struct {
    const float *input;
    const qtts_q4_view *w;
    int32_t k_start, k_end;
    float *partial;
} gemv_job;

static void *gemv_thread(void *arg) {
    gemv_job *j = (gemv_job *)arg;
    gemv_q4_inner(j->input, j->w->packed, j->w->scales, j->w->n, j->k_start, j->k_end, j->partial);
    return NULL;
}

/* gemv_q4, src/gemv.rs:263-309: split-K over available_parallelism() OS
 * threads spawned per call when k*n >= 4e6; partials summed in thread order. */
void qor_gemv(const float *input, const qtts_q4_view *w, float *out, int32_t nthreads) {
    const int32_t k = w->k, n = w->n;
    int32_t num_threads = 1;
    if ((int64_t)k * n >= 4000000) num_threads = nthreads > 0 ? nthreads : qor_available_parallelism();
    memset(out, 0, sizeof(float) * (size_t)n);
    if (num_threads <= 1) {
        gemv_q4_inner(input, w->packed, w->scales, n, 0, k, out);
        return;
    }
    const int32_t chunk_k = (k + num_threads - 1) / num_threads;
    float *partials = (float *)xcalloc((size_t)num_threads * n, sizeof(float));
    pthread_t *th = (pthread_t *)xcalloc((size_t)num_threads, sizeof(pthread_t));
    gemv_job *jobs = (gemv_job *)xcalloc((size_t)num_threads, sizeof(gemv_job));
    for (int32_t t = 0; t < num_threads; t++) {
        int32_t ks = t * chunk_k, ke = (t + 1) * chunk_k;
        if (ke > k) ke = k;
        jobs[t] = (gemv_job){input, w, ks, ke, partials + (size_t)t * n};
        if (pthread_create(&th[t], NULL, gemv_thread, &jobs[t]) != 0) {
            fprintf(stderr, "oracle: pthread_create failed\n");
            abort();
        }
    }
    for (int32_t t = 0; t < num_threads; t++) {
        pthread_join(th[t], NULL);
        const float *p = partials + (size_t)t * n;
        for (int32_t j = 0; j < n; j++) out[j] += p[j];
    }
    free(jobs);
    free(th);
    free(partials);
}

typedef struct {
    const float *x;
    const qtts_q4_view *w;
    int32_t t_start, t_end;
    float *out;
} gemm_job;

static void *gemm_thread(void *arg) {
    gemm_job *j = (gemm_job *)arg;
    const int32_t k = j->w->k, n = j->w->n;
    for (int32_t t = j->t_start; t < j->t_end; t++)
        gemv_q4_inner(j->x + (size_t)t * k, j->w->packed, j->w->scales, n, 0, k, j->out + (size_t)t * n);
    return NULL;
}

/* gemm_q4, src/gemv.rs:311-375: one full-K gemv_q4_inner per row; rows are
 * split over threads when k*n >= 4e6 and seq_len > 1. */
void qor_gemm(const float *x, int32_t seq_len, const qtts_q4_view *w, float *out, int32_t nthreads) {
    const int32_t k = w->k, n = w->n;
    int32_t num_threads = 1;
    if ((int64_t)k * n >= 4000000 && seq_len > 1) num_threads = nthreads > 0 ? nthreads : qor_available_parallelism();
    memset(out, 0, sizeof(float) * (size_t)seq_len * n);
    if (num_threads <= 1 || seq_len <= 1) {
        gemm_job j = {x, w, 0, seq_len, out};
        gemm_thread(&j);
        return;
    }
    const int32_t chunk = (seq_len + num_threads - 1) / num_threads;
    pthread_t *th = (pthread_t *)xcalloc((size_t)num_threads, sizeof(pthread_t));
    gemm_job *jobs = (gemm_job *)xcalloc((size_t)num_threads, sizeof(gemm_job));
    int32_t used = 0;
    for (int32_t t = 0; t < num_threads; t++) {
        int32_t ts = t * chunk, te = (t + 1) * chunk;
        if (ts >= seq_len) break;
        if (te > seq_len) te = seq_len;
        jobs[t] = (gemm_job){x, w, ts, te, out};
        pthread_create(&th[t], NULL, gemm_thread, &jobs[t]);
        used++;
    }
    for (int32_t t = 0; t < used; t++) pthread_join(th[t], NULL);
    free(jobs);
    free(th);
}

/* embed_lookup_q4, src/gemv.rs:377-400 (= src/talker.rs:119-150). */
void qor_embed_lookup(const qtts_q4_view *w, int32_t token_id, float *out) {
    const int32_t n = w->n;
    const int32_t groups_per_row = n / Q4_GROUP;
    const size_t scale_base = (size_t)token_id * groups_per_row;
    const size_t pack_base = (size_t)token_id * groups_per_row * (Q4_GROUP / 2);
    for (int32_t g = 0; g < groups_per_row; g++) {
        const float scale = qor_f16_to_f32(w->scales[scale_base + g]);
        const uint8_t *p = w->packed + pack_base + (size_t)g * (Q4_GROUP / 2);
        for (int32_t j = 0; j < Q4_GROUP / 2; j++) {
            const int32_t q0 = (int32_t)(p[j] & 0x0F) - 8;
            const int32_t q1 = (int32_t)((p[j] >> 4) & 0x0F) - 8;
            out[g * Q4_GROUP + j * 2] = scale * (float)q0;
            out[g * Q4_GROUP + j * 2 + 1] = scale * (float)q1;
        }
    }
}

/* rms_norm_f16, src/gemv.rs:406-417. */
void qor_rms_norm_f16(const float *x, const uint16_t *gamma, int32_t n, float *out) {
    float sum_sq = 0.0f;
    for (int32_t i = 0; i < n; i++) sum_sq += x[i] * x[i];
    const float inv_rms = 1.0f / sqrtf(sum_sq / (float)n + 1e-6f);
    for (int32_t i = 0; i < n; i++) out[i] = x[i] * inv_rms * qor_f16_to_f32(gamma[i]);
}

/* softmax_raw, src/gemv.rs:433-445. */
void qor_softmax_raw(float *scores, int32_t n) {
    float max_val = -INFINITY;
    for (int32_t i = 0; i < n; i++) max_val = fmaxf(max_val, scores[i]); /* f32::max drops NaN */
    float sum = 0.0f;
    for (int32_t i = 0; i < n; i++) {
        scores[i] = expf(scores[i] - max_val);
        sum += scores[i];
    }
    const float inv_sum = 1.0f / sum;
    for (int32_t i = 0; i < n; i++) scores[i] *= inv_sum;
}

/* silu, src/gemv.rs:447-451. */
float qor_silu(float x) { return x / (1.0f + expf(-x)); }

/* apply_qk_norm, src/talker.rs:86-99 and src/code_predictor.rs:84-93. */
void qor_qk_norm(float *data, int32_t num_heads, int32_t head_dim, const uint16_t *gamma) {
    for (int32_t h = 0; h < num_heads; h++) {
        float *d = data + (size_t)h * head_dim;
        float sum_sq = 0.0f;
        for (int32_t i = 0; i < head_dim; i++) sum_sq += d[i] * d[i];
        const float inv_rms = 1.0f / sqrtf(sum_sq / (float)head_dim + 1e-6f);
        for (int32_t i = 0; i < head_dim; i++) d[i] = d[i] * inv_rms * qor_f16_to_f32(gamma[i]);
    }
}

/* ------------------------------------------------------------------------ */
/* RoPE, src/rope.rs                                                         */
/* ------------------------------------------------------------------------ */

/* build_mrope_tables, src/rope.rs:11-41: freq_i = 1/theta^(2i/head_dim) in
 * double, angle = pos*freq, cos/sin in double then cast to float. */
void qor_build_rope_table(int32_t head_dim, int32_t max_pos, double theta, float *cos_table, float *sin_table) {
    const int32_t half = head_dim / 2;
    for (int32_t i = 0; i < half; i++) {
        const double freq = 1.0 / pow(theta, (double)(2 * i) / (double)head_dim);
        for (int32_t pos = 0; pos < max_pos; pos++) {
            const double angle = (double)pos * freq;
            cos_table[(size_t)pos * half + i] = (float)cos(angle);
            sin_table[(size_t)pos * half + i] = (float)sin(angle);
        }
    }
}

/* Split-half rotation, src/rope.rs:79-92 and src/code_predictor.rs:108-120. */
void qor_rope_split(float *data, int32_t num_heads, int32_t head_dim, int32_t pos, const float *cos_table,
                    const float *sin_table) {
    const int32_t half = head_dim / 2;
    const float *c = cos_table + (size_t)pos * half;
    const float *s = sin_table + (size_t)pos * half;
    for (int32_t h = 0; h < num_heads; h++) {
        float *d = data + (size_t)h * head_dim;
        for (int32_t i = 0; i < half; i++) {
            const float x1 = d[i], x2 = d[half + i];
            d[i] = x1 * c[i] - x2 * s[i];
            d[half + i] = x2 * c[i] + x1 * s[i];
        }
    }
}

/* ------------------------------------------------------------------------ */
/* KV cache, src/gemv.rs:75-86                                               */
/* ------------------------------------------------------------------------ */
struct qor_kv {
    int32_t layers, kv_heads, head_dim, capacity, len;
    float *k, *v; /* [layer][capacity][kv_heads*head_dim] */
};

qor_kv *qor_kv_new(int32_t num_layers, int32_t num_kv_heads, int32_t head_dim, int32_t capacity) {
    qor_kv *kv = (qor_kv *)xcalloc(1, sizeof(qor_kv));
    kv->layers = num_layers;
    kv->kv_heads = num_kv_heads;
    kv->head_dim = head_dim;
    kv->capacity = capacity;
    size_t cnt = (size_t)num_layers * capacity * num_kv_heads * head_dim;
    kv->k = (float *)xcalloc(cnt, sizeof(float));
    kv->v = (float *)xcalloc(cnt, sizeof(float));
    return kv;
}
void qor_kv_free(qor_kv *kv) {
    if (!kv) return;
    free(kv->k);
    free(kv->v);
    free(kv);
}
int32_t qor_kv_len(const qor_kv *kv) { return kv->len; }
void qor_kv_clear(qor_kv *kv) { kv->len = 0; }

static size_t kv_row(const qor_kv *kv) { return (size_t)kv->kv_heads * kv->head_dim; }
static float *kv_k(const qor_kv *kv, int32_t layer) { return kv->k + (size_t)layer * kv->capacity * kv_row(kv); }
static float *kv_v(const qor_kv *kv, int32_t layer) { return kv->v + (size_t)layer * kv->capacity * kv_row(kv); }

int32_t qor_kv_load(qor_kv *kv, const float *k, const float *v, int32_t len) {
    if (len < 0 || len > kv->capacity) return QTTS_ERANGE;
    const size_t row = kv_row(kv);
    for (int32_t l = 0; l < kv->layers; l++) {
        memcpy(kv_k(kv, l), k + (size_t)l * len * row, sizeof(float) * len * row);
        memcpy(kv_v(kv, l), v + (size_t)l * len * row, sizeof(float) * len * row);
    }
    kv->len = len;
    return QTTS_OK;
}
int32_t qor_kv_store(const qor_kv *kv, float *k, float *v) {
    const size_t row = kv_row(kv);
    for (int32_t l = 0; l < kv->layers; l++) {
        memcpy(k + (size_t)l * kv->len * row, kv_k(kv, l), sizeof(float) * kv->len * row);
        memcpy(v + (size_t)l * kv->len * row, kv_v(kv, l), sizeof(float) * kv->len * row);
    }
    return QTTS_OK;
}

/* GQA decode attention for one query row over positions [0, kv_len) of one
 * layer, src/talker.rs:304-331 (= src/code_predictor.rs:467-491 and the
 * causal loops of the prefills with kv_len = t1+1). */
static void attend(const float *q, const float *ck, const float *cv, int32_t kv_len, int32_t num_heads,
                   int32_t num_kv_heads, int32_t head_dim, float *attn_out, float *scores) {
    const float scale = 1.0f / sqrtf((float)head_dim);
    const int32_t kv_stride = num_kv_heads * head_dim;
    const int32_t groups = num_heads / num_kv_heads;
    for (int32_t h = 0; h < num_heads; h++) {
        const int32_t kv_h = h / groups;
        const float *qv = q + (size_t)h * head_dim;
        for (int32_t s = 0; s < kv_len; s++) {
            const float *kr = ck + (size_t)s * kv_stride + (size_t)kv_h * head_dim;
            float dot = 0.0f;
            for (int32_t d = 0; d < head_dim; d++) dot += qv[d] * kr[d];
            scores[s] = dot * scale;
        }
        qor_softmax_raw(scores, kv_len);
        float *o = attn_out + (size_t)h * head_dim;
        for (int32_t d = 0; d < head_dim; d++) o[d] = 0.0f;
        for (int32_t s = 0; s < kv_len; s++) {
            const float *vr = cv + (size_t)s * kv_stride + (size_t)kv_h * head_dim;
            const float sc = scores[s];
            for (int32_t d = 0; d < head_dim; d++) o[d] += sc * vr[d];
        }
    }
}

/* Shapes shared by the talker and predictor layer stacks. */
typedef struct {
    int32_t num_layers;
    const qtts_layer_view *layers;
    const uint16_t *final_norm_gamma;
    int32_t hidden, heads, kv_heads, head_dim, max_pos;
    float *rope_cos, *rope_sin;
    int32_t rope_skip_oob; /* predictor skips RoPE past the table (src/code_predictor.rs:107) */
} stack;

static void stack_rope(const stack *st, float *data, int32_t heads, int32_t pos) {
    if (pos >= st->max_pos) {
        if (st->rope_skip_oob) return;
    }
    qor_rope_split(data, heads, st->head_dim, pos, st->rope_cos, st->rope_sin);
}

/* One decode step through every layer: forward_with_embedding's layer loop,
 * src/talker.rs:274-350 (= decode_one_code_predictor_token,
 * src/code_predictor.rs:443-503).  x is updated in place. */
static int32_t stack_decode(const stack *st, float *x, qor_kv *kv, int32_t position, int32_t nthreads) {
    const int32_t hidden = st->hidden, hd = st->head_dim;
    const int32_t qd = st->heads * hd, kd = st->kv_heads * hd;
    const int32_t offset = kv->len;
    if (offset + 1 > kv->capacity) return QTTS_ERANGE;
    const int32_t inter = st->layers[0].gate_proj.n;
    float *x_norm = (float *)xcalloc((size_t)hidden, sizeof(float));
    float *q = (float *)xcalloc((size_t)qd, sizeof(float));
    float *kn = (float *)xcalloc((size_t)kd, sizeof(float));
    float *vn = (float *)xcalloc((size_t)kd, sizeof(float));
    float *attn = (float *)xcalloc((size_t)qd, sizeof(float));
    float *scores = (float *)xcalloc((size_t)offset + 1, sizeof(float));
    float *o = (float *)xcalloc((size_t)hidden, sizeof(float));
    float *gate = (float *)xcalloc((size_t)inter, sizeof(float));
    float *up = (float *)xcalloc((size_t)inter, sizeof(float));
    float *mid = (float *)xcalloc((size_t)inter, sizeof(float));
    for (int32_t i = 0; i < st->num_layers; i++) {
        const qtts_layer_view *lw = &st->layers[i];
        qor_rms_norm_f16(x, lw->input_norm_gamma, hidden, x_norm);
        qor_gemv(x_norm, &lw->q_proj, q, nthreads);
        qor_gemv(x_norm, &lw->k_proj, kn, nthreads);
        qor_gemv(x_norm, &lw->v_proj, vn, nthreads);
        qor_qk_norm(q, st->heads, hd, lw->q_norm);
        qor_qk_norm(kn, st->kv_heads, hd, lw->k_norm);
        /* talker: position argument (src/talker.rs:272); predictor: the
         * cache offset (src/code_predictor.rs:446,458). */
        const int32_t rpos = position >= 0 ? position : offset;
        stack_rope(st, q, st->heads, rpos);
        stack_rope(st, kn, st->kv_heads, rpos);
        float *ck = kv_k(kv, i), *cv = kv_v(kv, i);
        memcpy(ck + (size_t)offset * kd, kn, sizeof(float) * kd);
        memcpy(cv + (size_t)offset * kd, vn, sizeof(float) * kd);
        attend(q, ck, cv, offset + 1, st->heads, st->kv_heads, hd, attn, scores);
        qor_gemv(attn, &lw->o_proj, o, nthreads);
        for (int32_t j = 0; j < hidden; j++) x[j] += o[j];
        qor_rms_norm_f16(x, lw->post_attn_norm_gamma, hidden, x_norm);
        qor_gemv(x_norm, &lw->gate_proj, gate, nthreads);
        qor_gemv(x_norm, &lw->up_proj, up, nthreads);
        for (int32_t j = 0; j < inter; j++) mid[j] = qor_silu(gate[j]) * up[j];
        qor_gemv(mid, &lw->down_proj, o, nthreads);
        for (int32_t j = 0; j < hidden; j++) x[j] += o[j];
    }
    kv->len = offset + 1;
    free(x_norm); free(q); free(kn); free(vn); free(attn); free(scores);
    free(o); free(gate); free(up); free(mid);
    return QTTS_OK;
}

/* Multi-token prefill from an empty cache: prefill_talker_raw's layer loop,
 * src/talker.rs:373-457 (= prefill_code_predictor,
 * src/code_predictor.rs:347-425).  x is [seq_len][hidden], updated. */
static int32_t stack_prefill(const stack *st, float *x, int32_t seq_len, qor_kv *kv, int32_t nthreads) {
    const int32_t hidden = st->hidden, hd = st->head_dim;
    const int32_t qd = st->heads * hd, kd = st->kv_heads * hd;
    if (kv->len != 0) return QTTS_ESTATE;
    if (seq_len < 1) return QTTS_EINVAL;
    if (seq_len > kv->capacity) return QTTS_ERANGE;
    const int32_t inter = st->layers[0].gate_proj.n;
    const size_t S = (size_t)seq_len;
    float *x_norm = (float *)xcalloc(S * hidden, sizeof(float));
    float *q = (float *)xcalloc(S * qd, sizeof(float));
    float *kn = (float *)xcalloc(S * kd, sizeof(float));
    float *vn = (float *)xcalloc(S * kd, sizeof(float));
    float *attn = (float *)xcalloc(S * qd, sizeof(float));
    float *scores = (float *)xcalloc(S, sizeof(float));
    float *o = (float *)xcalloc(S * hidden, sizeof(float));
    float *gate = (float *)xcalloc(S * inter, sizeof(float));
    float *up = (float *)xcalloc(S * inter, sizeof(float));
    float *mid = (float *)xcalloc(S * inter, sizeof(float));
    for (int32_t i = 0; i < st->num_layers; i++) {
        const qtts_layer_view *lw = &st->layers[i];
        for (int32_t t = 0; t < seq_len; t++)
            qor_rms_norm_f16(x + t * (size_t)hidden, lw->input_norm_gamma, hidden, x_norm + t * (size_t)hidden);
        qor_gemm(x_norm, seq_len, &lw->q_proj, q, nthreads);
        qor_gemm(x_norm, seq_len, &lw->k_proj, kn, nthreads);
        qor_gemm(x_norm, seq_len, &lw->v_proj, vn, nthreads);
        for (int32_t t = 0; t < seq_len; t++) {
            qor_qk_norm(q + t * (size_t)qd, st->heads, hd, lw->q_norm);
            qor_qk_norm(kn + t * (size_t)kd, st->kv_heads, hd, lw->k_norm);
        }
        /* RoPE from start_pos 0 (src/talker.rs:395-402; predictor per token
         * at position t, src/code_predictor.rs:369-370). */
        for (int32_t t = 0; t < seq_len; t++) {
            stack_rope(st, q + t * (size_t)qd, st->heads, t);
            stack_rope(st, kn + t * (size_t)kd, st->kv_heads, t);
        }
        float *ck = kv_k(kv, i), *cv = kv_v(kv, i);
        memcpy(ck, kn, sizeof(float) * S * kd);
        memcpy(cv, vn, sizeof(float) * S * kd);
        for (int32_t t1 = 0; t1 < seq_len; t1++)
            attend(q + t1 * (size_t)qd, ck, cv, t1 + 1, st->heads, st->kv_heads, hd, attn + t1 * (size_t)qd, scores);
        qor_gemm(attn, seq_len, &lw->o_proj, o, nthreads);
        for (size_t j = 0; j < S * hidden; j++) x[j] += o[j];
        for (int32_t t = 0; t < seq_len; t++)
            qor_rms_norm_f16(x + t * (size_t)hidden, lw->post_attn_norm_gamma, hidden, x_norm + t * (size_t)hidden);
        qor_gemm(x_norm, seq_len, &lw->gate_proj, gate, nthreads);
        qor_gemm(x_norm, seq_len, &lw->up_proj, up, nthreads);
        for (size_t j = 0; j < S * inter; j++) mid[j] = qor_silu(gate[j]) * up[j];
        qor_gemm(mid, seq_len, &lw->down_proj, o, nthreads);
        for (size_t j = 0; j < S * hidden; j++) x[j] += o[j];
    }
    kv->len = seq_len;
    free(x_norm); free(q); free(kn); free(vn); free(attn); free(scores);
    free(o); free(gate); free(up); free(mid);
    return QTTS_OK;
}

/* ------------------------------------------------------------------------ */
/* Talker, src/talker.rs                                                     */
/* ------------------------------------------------------------------------ */
struct qor_talker {
    qtts_talker_view w;
    stack st;
};

qor_talker *qor_talker_new(const qtts_talker_view *w) {
    qor_talker *t = (qor_talker *)xcalloc(1, sizeof(qor_talker));
    t->w = *w;
    const int32_t half = w->head_dim / 2;
    t->st.num_layers = w->num_layers;
    t->st.layers = w->layers;
    t->st.final_norm_gamma = w->final_norm_gamma;
    t->st.hidden = w->hidden_size;
    t->st.heads = w->num_heads;
    t->st.kv_heads = w->num_kv_heads;
    t->st.head_dim = w->head_dim;
    t->st.max_pos = w->max_position;
    t->st.rope_cos = (float *)xcalloc((size_t)w->max_position * half, sizeof(float));
    t->st.rope_sin = (float *)xcalloc((size_t)w->max_position * half, sizeof(float));
    if (w->rope_cos && w->rope_sin) { /* a model file's tables (src/save.rs:84-85) */
        memcpy(t->st.rope_cos, w->rope_cos, (size_t)w->max_position * half * sizeof(float));
        memcpy(t->st.rope_sin, w->rope_sin, (size_t)w->max_position * half * sizeof(float));
    } else {
        qor_build_rope_table(w->head_dim, w->max_position, w->rope_theta, t->st.rope_cos, t->st.rope_sin);
    }
    t->st.rope_skip_oob = 0;
    return t;
}
void qor_talker_free(qor_talker *t) {
    if (!t) return;
    free(t->st.rope_cos);
    free(t->st.rope_sin);
    free(t);
}

/* forward_with_embedding, src/talker.rs:263-360. */
int32_t qor_forward_with_embedding(const qor_talker *t, const float *embedding, qor_kv *kv, int32_t position,
                                   float *out, int32_t nthreads) {
    const int32_t hidden = t->w.hidden_size;
    if (position < 0 || position >= t->w.max_position) return QTTS_ERANGE; /* rope.rs:73 would panic */
    float *x = (float *)xcalloc((size_t)hidden, sizeof(float));
    memcpy(x, embedding, sizeof(float) * hidden);
    int32_t rc = stack_decode(&t->st, x, kv, position, nthreads);
    if (rc == QTTS_OK) {
        qor_rms_norm_f16(x, t->w.final_norm_gamma, hidden, out);
        qor_gemv(out, &t->w.codec_head, out + hidden, nthreads);
    }
    free(x);
    return rc;
}

/* prefill_talker_raw, src/talker.rs:364-462. */
int32_t qor_prefill_talker_raw(const qor_talker *t, const float *x_in, int32_t seq_len, qor_kv *kv,
                               float *last_hidden, int32_t nthreads) {
    const int32_t hidden = t->w.hidden_size;
    if (seq_len > t->w.max_position) return QTTS_ERANGE;
    if (seq_len < 1) return QTTS_EINVAL;
    float *x = (float *)xcalloc((size_t)seq_len * hidden, sizeof(float));
    memcpy(x, x_in, sizeof(float) * (size_t)seq_len * hidden);
    int32_t rc = stack_prefill(&t->st, x, seq_len, kv, nthreads);
    if (rc == QTTS_OK) qor_rms_norm_f16(x + (size_t)(seq_len - 1) * hidden, t->w.final_norm_gamma, hidden, last_hidden);
    free(x);
    return rc;
}

int32_t qor_talker_hidden(const qor_talker *t) { return t->w.hidden_size; }
int32_t qor_talker_vocab(const qor_talker *t) { return t->w.codec_head.n; }
int32_t qor_talker_codec_rows(const qor_talker *t) { return t->w.codec_embedding.k; }

void qor_apply_codec_head(const qor_talker *t, const float *hidden, float *logits, int32_t nthreads) {
    qor_gemv(hidden, &t->w.codec_head, logits, nthreads);
}

void qor_embed_codec_token(const qor_talker *t, uint32_t token_id, float *out) {
    qor_embed_lookup(&t->w.codec_embedding, (int32_t)token_id, out);
}

/* ------------------------------------------------------------------------ */
/* Code Predictor, src/code_predictor.rs                                     */
/* ------------------------------------------------------------------------ */
struct qor_predictor {
    qtts_predictor_view w;
    stack st;
};

qor_predictor *qor_predictor_new(const qtts_predictor_view *w) {
    qor_predictor *p = (qor_predictor *)xcalloc(1, sizeof(qor_predictor));
    p->w = *w;
    /* The whole table, src/loader.rs:859-874 (max_position rows, 65536 for
     * the 1.7B model); positions past it skip the rotation
     * (src/code_predictor.rs:105-107). */
    const int32_t half = w->head_dim / 2;
    const int32_t rows = w->max_position;
    p->st.num_layers = w->num_layers;
    p->st.layers = w->layers;
    p->st.final_norm_gamma = w->final_norm_gamma;
    p->st.hidden = w->hidden_size;
    p->st.heads = w->num_heads;
    p->st.kv_heads = w->num_kv_heads;
    p->st.head_dim = w->head_dim;
    p->st.max_pos = rows;
    p->st.rope_cos = (float *)xcalloc((size_t)rows * half, sizeof(float));
    p->st.rope_sin = (float *)xcalloc((size_t)rows * half, sizeof(float));
    if (w->rope_cos && w->rope_sin) { /* a model file's tables (src/save.rs:135-136) */
        memcpy(p->st.rope_cos, w->rope_cos, (size_t)rows * half * sizeof(float));
        memcpy(p->st.rope_sin, w->rope_sin, (size_t)rows * half * sizeof(float));
    } else {
        qor_build_rope_table(w->head_dim, rows, w->rope_theta, p->st.rope_cos, p->st.rope_sin);
    }
    p->st.rope_skip_oob = 1;
    return p;
}
void qor_predictor_free(qor_predictor *p) {
    if (!p) return;
    free(p->st.rope_cos);
    free(p->st.rope_sin);
    free(p);
}

/* project_input, src/code_predictor.rs:51-61. */
static void project_input(const qor_predictor *p, const float *input, float *out, int32_t nthreads) {
    if (p->w.input_proj.k > 0) {
        qor_gemv(input, &p->w.input_proj, out, nthreads);
        if (p->w.input_proj_bias)
            for (int32_t j = 0; j < p->w.input_proj.n; j++) out[j] += p->w.input_proj_bias[j];
    } else {
        memcpy(out, input, sizeof(float) * p->w.hidden_size);
    }
}

/* sample_argmax, src/code_predictor.rs:328-334: Iterator::max_by keeps the
 * LAST of equal maxima; partial_cmp().unwrap() panics on NaN. */
int32_t qor_argmax(const float *logits, int32_t n, uint32_t *out) {
    if (n <= 0) {
        *out = 0;
        return QTTS_OK;
    }
    int32_t best = 0;
    for (int32_t i = 0; i < n; i++)
        if (logits[i] != logits[i]) return QTTS_ENAN;
    for (int32_t i = 1; i < n; i++)
        if (logits[i] >= logits[best]) best = i;
    *out = (uint32_t)best;
    return QTTS_OK;
}

/* generate_acoustic_codes, src/code_predictor.rs:218-273. */
int32_t qor_generate_acoustic_codes(const qor_predictor *p, const float *talker_hidden, const float *semantic_embed,
                                    qor_kv *kv, uint32_t *codes, int32_t nthreads) {
    const int32_t hidden = p->w.hidden_size;
    const int32_t groups = p->w.num_groups;
    qor_kv_clear(kv);
    float *x = (float *)xcalloc(2 * (size_t)hidden, sizeof(float));
    project_input(p, talker_hidden, x, nthreads);
    project_input(p, semantic_embed, x + hidden, nthreads);
    int32_t rc = stack_prefill(&p->st, x, 2, kv, nthreads);
    if (rc != QTTS_OK) {
        free(x);
        return rc;
    }
    float *h = (float *)xcalloc((size_t)hidden, sizeof(float));
    qor_rms_norm_f16(x + hidden, p->w.final_norm_gamma, hidden, h);
    int32_t vocab = p->w.lm_heads[0].n;
    float *logits = (float *)xcalloc((size_t)vocab, sizeof(float));
    qor_gemv(h, &p->w.lm_heads[0], logits, nthreads);
    rc = qor_argmax(logits, vocab, &codes[0]);
    const int32_t embed_dim = p->w.codec_embeddings[0].n;
    float *emb = (float *)xcalloc((size_t)embed_dim, sizeof(float));
    for (int32_t g = 1; g < groups && rc == QTTS_OK; g++) {
        qor_embed_lookup(&p->w.codec_embeddings[g - 1], (int32_t)codes[g - 1], emb);
        project_input(p, emb, x, nthreads);
        rc = stack_decode(&p->st, x, kv, -1, nthreads);
        if (rc != QTTS_OK) break;
        qor_rms_norm_f16(x, p->w.final_norm_gamma, hidden, h);
        vocab = p->w.lm_heads[g].n;
        qor_gemv(h, &p->w.lm_heads[g], logits, nthreads);
        rc = qor_argmax(logits, vocab, &codes[g]);
    }
    free(emb);
    free(logits);
    free(h);
    free(x);
    return rc;
}

/* predict_codes, src/code_predictor.rs:126-213: project_input, one decode
 * step at the cache offset (RoPE at the offset), the final norm, then every
 * lm_head on the same row. */
int32_t qor_predict_codes(const qor_predictor *p, const float *talker_hidden, qor_kv *kv, float *logits,
                          int32_t nthreads) {
    const int32_t hidden = p->w.hidden_size;
    float *x = (float *)xcalloc((size_t)hidden, sizeof(float));
    project_input(p, talker_hidden, x, nthreads);
    int32_t rc = stack_decode(&p->st, x, kv, -1, nthreads);
    if (rc == QTTS_OK) {
        float *h = (float *)xcalloc((size_t)hidden, sizeof(float));
        qor_rms_norm_f16(x, p->w.final_norm_gamma, hidden, h);
        size_t off = 0;
        for (int32_t g = 0; g < p->w.num_groups; g++) {
            qor_gemv(h, &p->w.lm_heads[g], logits + off, nthreads);
            off += (size_t)p->w.lm_heads[g].n;
        }
        free(h);
    }
    free(x);
    return rc;
}

/* get_acoustic_embeddings_sum, src/code_predictor.rs:280-293. */
void qor_get_acoustic_embeddings_sum(const qor_predictor *p, const uint32_t *codes, float *out) {
    const int32_t embed_dim = p->w.codec_embeddings[0].n;
    float *e = (float *)xcalloc((size_t)embed_dim, sizeof(float));
    for (int32_t j = 0; j < embed_dim; j++) out[j] = 0.0f;
    for (int32_t g = 0; g < p->w.num_groups; g++) {
        qor_embed_lookup(&p->w.codec_embeddings[g], (int32_t)codes[g], e);
        for (int32_t j = 0; j < embed_dim; j++) out[j] += e[j];
    }
    free(e);
}

/* ------------------------------------------------------------------------ */
/* Sampler and frame loop, src/generate_new.rs                               */
/* ------------------------------------------------------------------------ */

/* simple_rand, src/generate_new.rs:17-22: xorshift64 (13, 7, 17), then
 * (state as f32) / (u64::MAX as f32), both conversions round to nearest. */
float qor_simple_rand(uint64_t *state) {
    uint64_t s = *state;
    s ^= s << 13;
    s ^= s >> 7;
    s ^= s << 17;
    *state = s;
    return (float)s / (float)UINT64_MAX;
}

typedef struct {
    float v;
    int32_t i;
} scored;

/* sort_by(|a, b| b.1.partial_cmp(&a.1)) is stable: descending value, equal
 * values in index order. */
static int scored_cmp(const void *a, const void *b) {
    const scored *x = (const scored *)a, *y = (const scored *)b;
    if (x->v > y->v) return -1;
    if (x->v < y->v) return 1;
    return (x->i > y->i) - (x->i < y->i);
}

/* sample_token, src/generate_new.rs:329-391. */
int32_t qor_sample_token(const float *logits, int32_t vocab, const qtts_sampler *params, const uint32_t *prev_tokens,
                         int32_t n_prev, uint64_t *rng, uint32_t *token) {
    float *s = (float *)xcalloc((size_t)vocab, sizeof(float));
    memcpy(s, logits, sizeof(float) * vocab);
    if (params->repetition_penalty != 1.0f) {
        for (int32_t i = 0; i < n_prev; i++) {
            const uint32_t t = prev_tokens[i];
            if (t < (uint32_t)vocab) {
                if (s[t] > 0.0f)
                    s[t] /= params->repetition_penalty;
                else
                    s[t] *= params->repetition_penalty;
            }
        }
    }
    if (params->greedy) {
        int32_t rc = qor_argmax(s, vocab, token);
        free(s);
        return rc;
    }
    if (params->temperature != 1.0f)
        for (int32_t i = 0; i < vocab; i++) s[i] /= params->temperature;
    float max_score = -INFINITY;
    for (int32_t i = 0; i < vocab; i++) max_score = fmaxf(max_score, s[i]);
    for (int32_t i = 0; i < vocab; i++) s[i] = expf(s[i] - max_score);
    float sum = 0.0f;
    for (int32_t i = 0; i < vocab; i++) sum += s[i];
    for (int32_t i = 0; i < vocab; i++) s[i] /= sum;
    if (params->top_k > 0 && params->top_k < vocab) {
        scored *idx = (scored *)xcalloc((size_t)vocab, sizeof(scored));
        for (int32_t i = 0; i < vocab; i++) {
            if (s[i] != s[i]) { /* partial_cmp(NaN).unwrap() panics */
                free(idx);
                free(s);
                return QTTS_ENAN;
            }
            idx[i].v = s[i];
            idx[i].i = i;
        }
        qsort(idx, (size_t)vocab, sizeof(scored), scored_cmp);
        for (int32_t r = params->top_k; r < vocab; r++) s[idx[r].i] = 0.0f;
        free(idx);
        float sum2 = 0.0f;
        for (int32_t i = 0; i < vocab; i++) sum2 += s[i];
        if (sum2 > 0.0f)
            for (int32_t i = 0; i < vocab; i++) s[i] /= sum2;
    }
    const float r = qor_simple_rand(rng);
    float cumsum = 0.0f;
    *token = 0;
    for (int32_t i = 0; i < vocab; i++) {
        cumsum += s[i];
        if (r < cumsum) {
            *token = (uint32_t)i;
            break;
        }
    }
    free(s);
    return QTTS_OK;
}

/* generate::sample_top_k, src/generate.rs:50-84 (the legacy loop's sampler):
 * greedy (last of equal maxima) when temperature <= 0; else the top_k
 * logits in descending order (the reference's sort_unstable_by leaves equal
 * logits in no fixed order: here equal logits go by ascending index),
 * p_i = expf((l_i - l_0) / T) summed in that order, divided by the sum, and
 * the first i in that order with r < cumsum, else the k-th index.  NaN is
 * QTTS_ENAN (partial_cmp().unwrap()); top_k < 1 is QTTS_EINVAL (an empty
 * top list panics at indices[0]). */
int32_t qor_sample_top_k(const float *logits, int32_t vocab, float temperature, int32_t top_k, uint64_t *rng,
                         uint32_t *token) {
    for (int32_t i = 0; i < vocab; i++)
        if (logits[i] != logits[i]) return QTTS_ENAN;
    if (temperature <= 0.0f) return qor_argmax(logits, vocab, token);
    if (top_k < 1 || vocab < 1) return QTTS_EINVAL;
    const int32_t k = top_k < vocab ? top_k : vocab;
    scored *idx = (scored *)xcalloc((size_t)vocab, sizeof(scored));
    for (int32_t i = 0; i < vocab; i++) {
        idx[i].v = logits[i];
        idx[i].i = i;
    }
    qsort(idx, (size_t)vocab, sizeof(scored), scored_cmp);
    float *probs = (float *)xcalloc((size_t)k, sizeof(float));
    const float max_logit = idx[0].v;
    float sum = 0.0f;
    for (int32_t i = 0; i < k; i++) probs[i] = expf((idx[i].v - max_logit) / temperature);
    for (int32_t i = 0; i < k; i++) sum += probs[i];
    for (int32_t i = 0; i < k; i++) probs[i] /= sum;
    const float r = qor_simple_rand(rng);
    float cumsum = 0.0f;
    *token = (uint32_t)idx[k - 1].i;
    for (int32_t i = 0; i < k; i++) {
        cumsum += probs[i];
        if (r < cumsum) {
            *token = (uint32_t)idx[i].i;
            break;
        }
    }
    free(probs);
    free(idx);
    return QTTS_OK;
}

/* The frame loop of generate_speech, src/generate_new.rs:229-300. */
int32_t qor_generate_codes(const qor_talker *t, const qor_predictor *p, qor_kv *talker_kv, qor_kv *predictor_kv,
                           const float *last_hidden_in, const float *logits_in, int32_t position,
                           const float *trailing_text, int32_t trailing_len, const float *tts_pad_embed,
                           const qtts_loop_params *params, uint64_t seed, uint32_t *codes, int32_t *n_frames,
                           int32_t nthreads) {
    const int32_t hidden = t->w.hidden_size;
    const int32_t vocab = t->w.codec_head.n;
    const int32_t max_codes = params->max_codes;
    const int32_t groups = (params->talker_only || !p) ? 0 : p->w.num_groups;
    uint32_t prev_tokens[16] = {0};
    uint64_t rng = seed;
    float *last_hidden = (float *)xcalloc((size_t)hidden, sizeof(float));
    float *result = (float *)xcalloc((size_t)hidden + vocab, sizeof(float));
    float *semantic = (float *)xcalloc((size_t)hidden, sizeof(float));
    float *acoustic_sum = (float *)xcalloc((size_t)hidden, sizeof(float));
    memcpy(last_hidden, last_hidden_in, sizeof(float) * hidden);
    memcpy(result + hidden, logits_in, sizeof(float) * vocab);
    uint32_t acoustic[16];
    int32_t rc = QTTS_OK, frame = 0;
    *n_frames = 0;
    for (frame = 0; frame < max_codes; frame++) {
        uint32_t semantic_token = 0;
        rc = qor_sample_token(result + hidden, vocab, &params->sampler, prev_tokens, 16, &rng, &semantic_token);
        if (rc != QTTS_OK) break;
        if (params->stop_on_eos && semantic_token == params->codec_eos_id) break;
        codes[(size_t)0 * max_codes + frame] = semantic_token;
        prev_tokens[0] = semantic_token;
        if (semantic_token >= (uint32_t)t->w.codec_embedding.k) {
            rc = QTTS_ERANGE;
            break;
        }
        qor_embed_codec_token(t, semantic_token, semantic);
        if (groups > 0) {
            rc = qor_generate_acoustic_codes(p, last_hidden, semantic, predictor_kv, acoustic, nthreads);
            if (rc != QTTS_OK) break;
            for (int32_t g = 0; g < groups; g++) {
                codes[(size_t)(g + 1) * max_codes + frame] = acoustic[g];
                prev_tokens[g + 1] = acoustic[g];
            }
            qor_get_acoustic_embeddings_sum(p, acoustic, acoustic_sum);
            for (int32_t j = 0; j < hidden; j++) semantic[j] += acoustic_sum[j];
            const float *text = frame < trailing_len ? trailing_text + (size_t)frame * hidden : tts_pad_embed;
            for (int32_t j = 0; j < hidden; j++) semantic[j] += text[j];
        }
        rc = qor_forward_with_embedding(t, semantic, talker_kv, position, result, nthreads);
        if (rc != QTTS_OK) break;
        memcpy(last_hidden, result, sizeof(float) * hidden);
        position += 1;
        *n_frames = frame + 1;
    }
    if (rc == QTTS_OK) *n_frames = frame;
    free(last_hidden);
    free(result);
    free(semantic);
    free(acoustic_sum);
    return rc;
}
