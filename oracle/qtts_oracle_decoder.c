/*
 * qtts_oracle_decoder.c — CPU restatement of the speech decoder
 * (src/decoder.rs, src/conv.rs).
 *
 * TEST INFRASTRUCTURE ONLY: the reference the decoder's parity tests compare
 * the HIP library against.  Nothing in the product library links it.
 *
 * Every sum keeps the reference's order: the f32 GEMVs accumulate over k
 * ascending (skipping zero inputs), convolutions over (in channel, tap) per
 * output, the transposed convolution over (in channel, input position, tap),
 * norms and softmax sequentially.  The reference's thread splits of the
 * convolutions are over output channels, so no result depends on the thread
 * count; the oracle splits the same way.
 */
#include <math.h>
#include <pthread.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#include "qtts_oracle.h"

static void *dcalloc(size_t n, size_t sz) {
    void *p = calloc(n ? n : 1, sz);
    if (!p) abort();
    return p;
}

/* f32_gemv / f32_gemv_bias, src/decoder.rs:527-553. */
static void f32_gemv(const float *in, const float *w, int32_t k, int32_t n, const float *bias, float *out) {
    for (int32_t j = 0; j < n; j++) out[j] = bias ? bias[j] : 0.0f;
    for (int32_t ki = 0; ki < k; ki++) {
        const float iv = in[ki];
        if (iv == 0.0f) continue;
        const float *row = w + (size_t)ki * n;
        for (int32_t j = 0; j < n; j++) out[j] += iv * row[j];
    }
}

/* rms_norm_f32, src/decoder.rs:515-525. */
static void rms_norm_f32(const float *x, const float *gamma, float eps, int32_t n, float *out) {
    float ss = 0.0f;
    for (int32_t i = 0; i < n; i++) ss += x[i] * x[i];
    const float inv = 1.0f / sqrtf(ss / (float)n + eps);
    for (int32_t i = 0; i < n; i++) out[i] = x[i] * inv * gamma[i];
}

/* apply_rope_split_half, src/decoder.rs:556-578: no rotation past the table. */
static void rope_split_half(float *data, int32_t heads, int32_t hd, int32_t pos, const float *cs, const float *sn,
                            int32_t rows) {
    const int32_t half = hd / 2;
    if (pos >= rows) return;
    const float *c = cs + (size_t)pos * half, *s = sn + (size_t)pos * half;
    for (int32_t h = 0; h < heads; h++) {
        float *b = data + (size_t)h * hd;
        for (int32_t i = 0; i < half; i++) {
            const float x0 = b[i], x1 = b[half + i];
            b[i] = x0 * c[i] - x1 * s[i];
            b[half + i] = x1 * c[i] + x0 * s[i];
        }
    }
}

/* layer_norm_channel_first, src/decoder.rs:580-602. */
static void layer_norm_cf(const float *in, const float *g, const float *b, int32_t ch, int32_t len, float eps,
                          float *out) {
    for (int32_t t = 0; t < len; t++) {
        float mean = 0.0f;
        for (int32_t c = 0; c < ch; c++) mean += in[(size_t)c * len + t];
        mean /= (float)ch;
        float var = 0.0f;
        for (int32_t c = 0; c < ch; c++) {
            const float d = in[(size_t)c * len + t] - mean;
            var += d * d;
        }
        const float inv = 1.0f / sqrtf(var / (float)ch + eps);
        for (int32_t c = 0; c < ch; c++)
            out[(size_t)c * len + t] = (in[(size_t)c * len + t] - mean) * inv * g[c] + b[c];
    }
}

/* gelu, src/conv.rs:453-455 (the tanh form the reference evaluates). */
static float gelu(float x) { return x * 0.5f * (1.0f + tanhf(x * 0.7071067811865476f)); }

/* ---- convolutions: a parallel-for over output channels ------------------ */
typedef struct {
    int kind; /* 0 causal, 1 transposed, 2 depthwise, 3 snake */
    const float *in;
    const qtts_conv_view *w;
    const float *alpha, *beta;
    int32_t in_len, out_len, c0, c1;
    float *out;
} conv_job;

/* causal_conv1d_range, src/conv.rs:151-184. */
static void causal_range(const conv_job *j) {
    const qtts_conv_view *w = j->w;
    const int32_t pad = (w->kernel_size - 1) * w->dilation, ick = w->in_channels * w->kernel_size;
    for (int32_t oc = j->c0; oc < j->c1; oc++) {
        for (int32_t o = 0; o < j->out_len; o++) {
            float sum = w->bias[oc];
            for (int32_t ic = 0; ic < w->in_channels; ic++) {
                const float *row = j->in + (size_t)ic * j->in_len;
                const float *wr = w->weight + (size_t)oc * ick + (size_t)ic * w->kernel_size;
                for (int32_t k = 0; k < w->kernel_size; k++) {
                    const int32_t p = o + k * w->dilation;
                    if (p >= pad && p - pad < j->in_len) sum += row[p - pad] * wr[k];
                }
            }
            j->out[(size_t)oc * j->out_len + o] = sum;
        }
    }
}

/* conv_transpose1d_range, src/conv.rs:235-268. */
static void transposed_range(const conv_job *j) {
    const qtts_conv_view *w = j->w;
    for (int32_t oc = j->c0; oc < j->c1; oc++) {
        float *orow = j->out + (size_t)oc * j->out_len;
        for (int32_t o = 0; o < j->out_len; o++) orow[o] = w->bias[oc];
        for (int32_t ic = 0; ic < w->in_channels; ic++) {
            const float *row = j->in + (size_t)ic * j->in_len;
            const float *wb = w->weight + ((size_t)ic * w->out_channels + oc) * w->kernel_size;
            for (int32_t i = 0; i < j->in_len; i++) {
                const float v = row[i];
                if (v == 0.0f) continue;
                for (int32_t k = 0; k < w->kernel_size; k++) {
                    const int64_t op = (int64_t)i * w->stride + k - w->padding;
                    if (op >= 0 && op < j->out_len) orow[op] += v * wb[k];
                }
            }
        }
    }
}

/* dw_conv1d_range, src/conv.rs:317-345: causal, padding kernel_size - 1. */
static void depthwise_range(const conv_job *j) {
    const qtts_conv_view *w = j->w;
    const int32_t pad = w->kernel_size - 1;
    for (int32_t c = j->c0; c < j->c1; c++) {
        for (int32_t o = 0; o < j->out_len; o++) {
            float sum = w->bias[c];
            for (int32_t k = 0; k < w->kernel_size; k++) {
                const int32_t p = o + k;
                if (p >= pad && p - pad < j->in_len)
                    sum += j->in[(size_t)c * j->in_len + p - pad] * w->weight[(size_t)c * w->kernel_size + k];
            }
            j->out[(size_t)c * j->out_len + o] = sum;
        }
    }
}

/* snake_beta_range, src/conv.rs:381-400: x + exp(-beta) * sin(exp(alpha) x)^2. */
static void snake_range(const conv_job *j) {
    for (int32_t c = j->c0; c < j->c1; c++) {
        const float a = expf(j->alpha[c]), inv_b = expf(-j->beta[c]);
        for (int32_t t = 0; t < j->in_len; t++) {
            const float x = j->in[(size_t)c * j->in_len + t];
            const float s = sinf(a * x);
            j->out[(size_t)c * j->in_len + t] = x + inv_b * s * s;
        }
    }
}

static void *job_main(void *arg) {
    const conv_job *j = (const conv_job *)arg;
    switch (j->kind) {
        case 0: causal_range(j); break;
        case 1: transposed_range(j); break;
        case 2: depthwise_range(j); break;
        default: snake_range(j); break;
    }
    return NULL;
}

static void run_channels(conv_job proto, int32_t channels, int32_t nthreads) {
    if (nthreads <= 0) nthreads = qor_available_parallelism();
    if (nthreads > channels) nthreads = channels;
    if (nthreads <= 1) {
        proto.c0 = 0;
        proto.c1 = channels;
        job_main(&proto);
        return;
    }
    pthread_t th[256];
    conv_job jobs[256];
    if (nthreads > 256) nthreads = 256;
    const int32_t chunk = (channels + nthreads - 1) / nthreads;
    int32_t n = 0;
    for (int32_t t = 0; t < nthreads; t++) {
        jobs[t] = proto;
        jobs[t].c0 = t * chunk;
        jobs[t].c1 = (t + 1) * chunk < channels ? (t + 1) * chunk : channels;
        if (jobs[t].c0 >= jobs[t].c1) break;
        pthread_create(&th[t], NULL, job_main, &jobs[t]);
        n++;
    }
    for (int32_t t = 0; t < n; t++) pthread_join(th[t], NULL);
}

static float *causal_conv(const float *in, int32_t len, const qtts_conv_view *w, int32_t nt) {
    float *out = (float *)dcalloc((size_t)w->out_channels * len, sizeof(float));
    conv_job j = {0, in, w, NULL, NULL, len, len, 0, 0, out};
    run_channels(j, w->out_channels, nt);
    return out;
}

/* conv_transpose1d then the causal right crop of kernel_size - stride
 * (src/decoder.rs:430-444, 462-474). */
static float *transposed_conv_cropped(const float *in, int32_t len, const qtts_conv_view *w, int32_t *out_len,
                                      int32_t nt) {
    const int32_t full = (len - 1) * w->stride - 2 * w->padding + w->kernel_size;
    float *o = (float *)dcalloc((size_t)w->out_channels * full, sizeof(float));
    conv_job j = {1, in, w, NULL, NULL, len, full, 0, 0, o};
    run_channels(j, w->out_channels, nt);
    const int32_t crop = w->kernel_size - w->stride;
    if (crop <= 0) {
        *out_len = full;
        return o;
    }
    const int32_t cl = full - crop;
    float *c = (float *)dcalloc((size_t)w->out_channels * cl, sizeof(float));
    for (int32_t ch = 0; ch < w->out_channels; ch++) memcpy(c + (size_t)ch * cl, o + (size_t)ch * full, cl * 4);
    free(o);
    *out_len = cl;
    return c;
}

static float *snake(const float *in, int32_t ch, int32_t len, const float *alpha, const float *beta, int32_t nt) {
    float *out = (float *)dcalloc((size_t)ch * len, sizeof(float));
    conv_job j = {3, in, NULL, alpha, beta, len, len, 0, 0, out};
    run_channels(j, ch, nt);
    return out;
}

/* codebook_lookup, src/decoder.rs:142-189: [vq_dim][T]. */
static float *codebook_lookup(const qtts_decoder_view *w, const uint32_t *codes, int32_t T, int32_t ld) {
    const int32_t cd = w->codebook_dim, vq = w->vq_dim;
    float *out = (float *)dcalloc((size_t)vq * T, sizeof(float));
    float *proj = (float *)dcalloc((size_t)vq, sizeof(float));
    float *sum = (float *)dcalloc((size_t)cd, sizeof(float));
    for (int32_t t = 0; t < T; t++) {
        const float *e = w->first_codebook + (size_t)codes[t] * cd;
        f32_gemv(e, w->first_output_proj, cd, vq, NULL, proj);
        for (int32_t c = 0; c < vq; c++) out[(size_t)c * T + t] += proj[c];
    }
    for (int32_t t = 0; t < T; t++) {
        for (int32_t d = 0; d < cd; d++) sum[d] = 0.0f;
        for (int32_t g = 0; g < w->num_rest; g++) {
            const float *e = w->rest_codebooks[g] + (size_t)codes[(size_t)(g + 1) * ld + t] * cd;
            for (int32_t d = 0; d < cd; d++) sum[d] += e[d];
        }
        f32_gemv(sum, w->rest_output_proj, cd, vq, NULL, proj);
        for (int32_t c = 0; c < vq; c++) out[(size_t)c * T + t] += proj[c];
    }
    free(proj);
    free(sum);
    return out;
}

/* Causal sliding-window attention of row t (src/decoder.rs:262-300): each
 * head attends to positions max(0, t+1-window) .. t; scores q.k * scale in
 * dimension order, softmax_raw, then sum_s p_s v_s in position order.  q, k,
 * v are [T][heads*hd]; sc holds window+1 floats; ao receives [heads*hd]. */
static void window_attention_row(const float *q, const float *k, const float *v, int32_t t, int32_t heads,
                                 int32_t hd, int32_t window, float scale, float *sc, float *ao) {
    const int32_t ad = heads * hd;
    const int32_t start = t + 1 > window ? t + 1 - window : 0;
    const int32_t n = t + 1 - start;
    for (int32_t i = 0; i < ad; i++) ao[i] = 0.0f;
    for (int32_t h = 0; h < heads; h++) {
        const float *qh = q + (size_t)t * ad + (size_t)h * hd;
        for (int32_t s = 0; s < n; s++) {
            const float *kh = k + (size_t)(start + s) * ad + (size_t)h * hd;
            float dot = 0.0f;
            for (int32_t d = 0; d < hd; d++) dot += qh[d] * kh[d];
            sc[s] = dot * scale;
        }
        qor_softmax_raw(sc, n);
        for (int32_t s = 0; s < n; s++) {
            const float *vh = v + (size_t)(start + s) * ad + (size_t)h * hd;
            for (int32_t d = 0; d < hd; d++) ao[(size_t)h * hd + d] += sc[s] * vh[d];
        }
    }
}

/* decoder_transformer, src/decoder.rs:195-330: [latent][T] -> [latent][T]. */
static float *decoder_transformer(const qtts_decoder_view *w, const float *x_ch, int32_t T) {
    const int32_t hid = w->hidden_size, ad = w->num_heads * w->head_dim, in_dim = w->pre_conv.out_channels;
    const int32_t inter = w->intermediate_size, hd = w->head_dim;
    float *xr = (float *)dcalloc((size_t)T * in_dim, sizeof(float));
    for (int32_t c = 0; c < in_dim; c++)
        for (int32_t t = 0; t < T; t++) xr[(size_t)t * in_dim + c] = x_ch[(size_t)c * T + t];
    float *x = (float *)dcalloc((size_t)T * hid, sizeof(float));
    for (int32_t t = 0; t < T; t++) f32_gemv(xr + (size_t)t * in_dim, w->tf_input_w, in_dim, hid, w->tf_input_b, x + (size_t)t * hid);
    float *q = (float *)dcalloc((size_t)T * ad, sizeof(float));
    float *k = (float *)dcalloc((size_t)T * ad, sizeof(float));
    float *v = (float *)dcalloc((size_t)T * ad, sizeof(float));
    float *xn = (float *)dcalloc((size_t)hid, sizeof(float));
    float *ao = (float *)dcalloc((size_t)ad, sizeof(float));
    float *tmp = (float *)dcalloc((size_t)(hid > inter ? hid : inter), sizeof(float));
    float *g = (float *)dcalloc((size_t)inter, sizeof(float));
    float *u = (float *)dcalloc((size_t)inter, sizeof(float));
    float *sc = (float *)dcalloc((size_t)(w->sliding_window > 0 ? w->sliding_window : 1) + (size_t)T, sizeof(float));
    const float scale = 1.0f / sqrtf((float)hd);
    for (int32_t l = 0; l < w->num_layers; l++) {
        const qtts_dec_layer_view *L = &w->layers[l];
        for (int32_t t = 0; t < T; t++) {
            rms_norm_f32(x + (size_t)t * hid, L->input_norm, 1e-5f, hid, xn);
            f32_gemv(xn, L->q_proj, hid, ad, NULL, q + (size_t)t * ad);
            f32_gemv(xn, L->k_proj, hid, ad, NULL, k + (size_t)t * ad);
            f32_gemv(xn, L->v_proj, hid, ad, NULL, v + (size_t)t * ad);
        }
        for (int32_t t = 0; t < T; t++) {
            rope_split_half(q + (size_t)t * ad, w->num_heads, hd, t, w->rope_cos, w->rope_sin, w->rope_rows);
            rope_split_half(k + (size_t)t * ad, w->num_heads, hd, t, w->rope_cos, w->rope_sin, w->rope_rows);
        }
        for (int32_t t = 0; t < T; t++) {
            window_attention_row(q, k, v, t, w->num_heads, hd, w->sliding_window, scale, sc, ao);
            f32_gemv(ao, L->o_proj, ad, hid, NULL, tmp);
            for (int32_t j = 0; j < hid; j++) x[(size_t)t * hid + j] += tmp[j] * L->attn_scale[j];
        }
        for (int32_t t = 0; t < T; t++) {
            rms_norm_f32(x + (size_t)t * hid, L->post_attn_norm, 1e-5f, hid, xn);
            f32_gemv(xn, L->gate_proj, hid, inter, NULL, g);
            f32_gemv(xn, L->up_proj, hid, inter, NULL, u);
            for (int32_t j = 0; j < inter; j++) g[j] = (g[j] / (1.0f + expf(-g[j]))) * u[j];
            f32_gemv(g, L->down_proj, inter, hid, NULL, tmp);
            for (int32_t j = 0; j < hid; j++) x[(size_t)t * hid + j] += tmp[j] * L->mlp_scale[j];
        }
    }
    for (int32_t t = 0; t < T; t++) {
        rms_norm_f32(x + (size_t)t * hid, w->tf_norm, 1e-5f, hid, xn);
        memcpy(x + (size_t)t * hid, xn, (size_t)hid * 4);
    }
    float *orow = (float *)dcalloc((size_t)T * in_dim, sizeof(float));
    for (int32_t t = 0; t < T; t++)
        f32_gemv(x + (size_t)t * hid, w->tf_output_w, hid, in_dim, w->tf_output_b, orow + (size_t)t * in_dim);
    float *out = (float *)dcalloc((size_t)T * in_dim, sizeof(float));
    for (int32_t c = 0; c < in_dim; c++)
        for (int32_t t = 0; t < T; t++) out[(size_t)c * T + t] = orow[(size_t)t * in_dim + c];
    free(xr); free(x); free(q); free(k); free(v); free(xn); free(ao); free(tmp); free(g); free(u); free(sc);
    free(orow);
    return out;
}

/* convnext_forward, src/decoder.rs:336-388. */
static float *convnext(const float *in, int32_t len, const qtts_upsample_view *st, int32_t nt) {
    const int32_t ch = st->channels, inner = st->inner_dim;
    float *dw = (float *)dcalloc((size_t)ch * len, sizeof(float));
    conv_job j = {2, in, &st->dw_conv, NULL, NULL, len, len, 0, 0, dw};
    run_channels(j, ch, nt);
    float *nrm = (float *)dcalloc((size_t)ch * len, sizeof(float));
    layer_norm_cf(dw, st->norm_w, st->norm_b, ch, len, 1e-5f, nrm);
    float *xt = (float *)dcalloc((size_t)(ch > inner ? ch : inner), sizeof(float));
    float *yt = (float *)dcalloc((size_t)(ch > inner ? ch : inner), sizeof(float));
    float *p1 = (float *)dcalloc((size_t)inner * len, sizeof(float));
    for (int32_t t = 0; t < len; t++) {
        for (int32_t c = 0; c < ch; c++) xt[c] = nrm[(size_t)c * len + t];
        f32_gemv(xt, st->pw1_w, ch, inner, st->pw1_b, yt);
        for (int32_t c = 0; c < inner; c++) p1[(size_t)c * len + t] = gelu(yt[c]);
    }
    float *out = (float *)dcalloc((size_t)ch * len, sizeof(float));
    for (int32_t t = 0; t < len; t++) {
        for (int32_t c = 0; c < inner; c++) xt[c] = p1[(size_t)c * len + t];
        f32_gemv(xt, st->pw2_w, inner, ch, st->pw2_b, yt);
        for (int32_t c = 0; c < ch; c++) out[(size_t)c * len + t] = in[(size_t)c * len + t] + st->gamma[c] * yt[c];
    }
    free(dw); free(nrm); free(xt); free(yt); free(p1);
    return out;
}

int64_t qor_decoder_num_samples(const qtts_decoder_view *w, int32_t frames) {
    if (frames <= 0) return 0;
    int64_t len = frames;
    for (int32_t i = 0; i < w->num_upsample; i++) {
        const qtts_conv_view *c = &w->upsample[i].conv_t;
        const int64_t full = (len - 1) * c->stride - 2 * c->padding + c->kernel_size;
        const int64_t crop = c->kernel_size - c->stride;
        len = crop > 0 ? full - crop : full;
    }
    for (int32_t b = 0; b < w->num_vocos_blocks; b++) {
        const qtts_conv_view *c = &w->vocos_blocks[b].upsample;
        const int64_t full = (len - 1) * c->stride - 2 * c->padding + c->kernel_size;
        const int64_t crop = c->kernel_size - c->stride;
        len = crop > 0 ? full - crop : full;
    }
    return len * w->output_conv.out_channels;
}

/* decode_to_audio, src/decoder.rs:394-509. */
int32_t qor_decode_to_audio(const qtts_decoder_view *w, const uint32_t *codes, int32_t frames, int32_t ld,
                            float *audio, int64_t capacity, int64_t *n_samples, int32_t nthreads) {
    *n_samples = 0;
    if (frames <= 0) return QTTS_OK;
    const int64_t need = qor_decoder_num_samples(w, frames);
    if (need > capacity) return QTTS_ERANGE;
    for (int32_t g = 0; g <= w->num_rest; g++)
        for (int32_t t = 0; t < frames; t++)
            if (codes[(size_t)g * ld + t] >= (uint32_t)w->codebook_size) return QTTS_ERANGE;
    float *vq = codebook_lookup(w, codes, frames, ld);
    float *sig = causal_conv(vq, frames, &w->pre_conv, nthreads);
    free(vq);
    float *tf = decoder_transformer(w, sig, frames);
    free(sig);
    sig = tf;
    int32_t len = frames, ch = w->pre_conv.out_channels;
    for (int32_t i = 0; i < w->num_upsample; i++) {
        const qtts_upsample_view *st = &w->upsample[i];
        int32_t nl;
        float *up = transposed_conv_cropped(sig, len, &st->conv_t, &nl, nthreads);
        free(sig);
        len = nl;
        ch = st->channels;
        sig = convnext(up, len, st, nthreads);
        free(up);
    }
    float *vi = causal_conv(sig, len, &w->vocos_init, nthreads);
    free(sig);
    sig = vi;
    ch = w->vocos_init.out_channels;
    for (int32_t b = 0; b < w->num_vocos_blocks; b++) {
        const qtts_vocos_block_view *vb = &w->vocos_blocks[b];
        float *s = snake(sig, vb->upsample.in_channels, len, vb->pre_snake_alpha, vb->pre_snake_beta, nthreads);
        free(sig);
        int32_t nl;
        sig = transposed_conv_cropped(s, len, &vb->upsample, &nl, nthreads);
        free(s);
        len = nl;
        ch = vb->upsample.out_channels;
        for (int32_t r = 0; r < vb->num_residuals; r++) {
            const qtts_vocos_residual_view *rv = &vb->residuals[r];
            float *a1 = snake(sig, ch, len, rv->act1_alpha, rv->act1_beta, nthreads);
            float *c1 = causal_conv(a1, len, &rv->conv1, nthreads);
            free(a1);
            float *a2 = snake(c1, ch, len, rv->act2_alpha, rv->act2_beta, nthreads);
            free(c1);
            float *c2 = causal_conv(a2, len, &rv->conv2, nthreads);
            free(a2);
            for (size_t i = 0; i < (size_t)ch * len; i++) c2[i] += sig[i];
            free(sig);
            sig = c2;
        }
    }
    const int32_t fch = w->output_conv.in_channels;
    float *fs = snake(sig, fch, len, w->final_snake_alpha, w->final_snake_beta, nthreads);
    free(sig);
    float *o = causal_conv(fs, len, &w->output_conv, nthreads);
    free(fs);
    const int64_t n = (int64_t)len * w->output_conv.out_channels;
    for (int64_t i = 0; i < n; i++) {
        float s = o[i];
        if (s < -1.0f) s = -1.0f;
        else if (s > 1.0f) s = 1.0f;
        audio[i] = s;
    }
    free(o);
    *n_samples = n;
    return QTTS_OK;
}

/* ---- Test hooks ----------------------------------------------------------
 * The decoder's primitives above, exported so that CPU tests can check each
 * against a closed form or a float64 brute force.  Layouts are the ones the
 * primitives use: channel-first [ch][len] signals, token-major [T][D] rows. */
void qor_dec_causal_conv(const float *in, int32_t len, const qtts_conv_view *w, float *out, int32_t nt) {
    float *o = causal_conv(in, len, w, nt);
    memcpy(out, o, (size_t)w->out_channels * len * sizeof(float));
    free(o);
}

int32_t qor_dec_transposed_conv(const float *in, int32_t len, const qtts_conv_view *w, float *out, int32_t nt) {
    int32_t ol = 0;
    float *o = transposed_conv_cropped(in, len, w, &ol, nt);
    memcpy(out, o, (size_t)w->out_channels * ol * sizeof(float));
    free(o);
    return ol;
}

void qor_dec_depthwise_conv(const float *in, int32_t len, const qtts_conv_view *w, float *out, int32_t nt) {
    conv_job j = {2, in, w, NULL, NULL, len, len, 0, 0, out};
    run_channels(j, w->out_channels, nt);
}

void qor_dec_snake(const float *in, int32_t ch, int32_t len, const float *alpha, const float *beta, float *out,
                   int32_t nt) {
    float *o = snake(in, ch, len, alpha, beta, nt);
    memcpy(out, o, (size_t)ch * len * sizeof(float));
    free(o);
}

float qor_dec_gelu(float x) { return gelu(x); }

void qor_dec_layer_norm_cf(const float *in, const float *g, const float *b, int32_t ch, int32_t len, float eps,
                           float *out) {
    layer_norm_cf(in, g, b, ch, len, eps, out);
}

void qor_dec_rms_norm(const float *x, const float *gamma, float eps, int32_t n, float *out) {
    rms_norm_f32(x, gamma, eps, n, out);
}

void qor_dec_rope(float *data, int32_t heads, int32_t hd, int32_t pos, const float *cs, const float *sn,
                  int32_t rows) {
    rope_split_half(data, heads, hd, pos, cs, sn, rows);
}

void qor_dec_window_attention(const float *q, const float *k, const float *v, int32_t T, int32_t heads, int32_t hd,
                              int32_t window, float *out) {
    float *sc = (float *)dcalloc((size_t)(window > 0 ? window : 1) + (size_t)T, sizeof(float));
    const float scale = 1.0f / sqrtf((float)hd);
    for (int32_t t = 0; t < T; t++)
        window_attention_row(q, k, v, t, heads, hd, window, scale, sc, out + (size_t)t * heads * hd);
    free(sc);
}

void qor_dec_codebook_lookup(const qtts_decoder_view *w, const uint32_t *codes, int32_t T, int32_t ld, float *out) {
    float *o = codebook_lookup(w, codes, T, ld);
    memcpy(out, o, (size_t)w->vq_dim * T * sizeof(float));
    free(o);
}
