/*
 * qtts_oracle_prompt.c — CPU restatement of the prompt assembly around the
 * per-code loop: embed_text_token (src/talker.rs:105-116), the role prefix and
 * TTS pad/BOS overlay (src/generate_new.rs:60-80), prefill_custom_voice
 * (src/generate_new.rs:84-188), build_trailing_text (src/generate_new.rs:
 * 314-326) and generate_speech from token ids to codes (src/generate_new.rs:
 * 191-300, without the tokenizer and the speech decoder).
 *
 * TEST INFRASTRUCTURE ONLY: the reference the prompt path's parity tests
 * compare the HIP library against.  Nothing in the product library links it.
 *
 * Arithmetic follows the reference step for step: the text projection is
 * gemv(fc1) then + bias, SiLU, gemv(fc2) then + bias; every combined row is
 * codec embedding + text row, added element by element.
 */
#include <stdlib.h>
#include <string.h>

#include "qtts_oracle.h"

/* Special tokens, src/generate_new.rs:24-36. */
enum {
    IM_START = 151644,
    ASSISTANT = 77091,
    NEWLINE = 198,
    TTS_PAD = 151671,
    TTS_BOS = 151672,
    TTS_EOS = 151673,
    CODEC_THINK = 2154,
    CODEC_THINK_BOS = 2156,
    CODEC_THINK_EOS = 2157,
    CODEC_PAD = 2148,
    CODEC_BOS = 2149
};

struct qor_text {
    qtts_text_view w;
    int32_t hidden; /* output width (fc2.n) */
};

qor_text *qor_text_new(const qtts_text_view *w) {
    qor_text *x = (qor_text *)calloc(1, sizeof(qor_text));
    if (!x) abort();
    x->w = *w;
    x->hidden = w->text_proj_fc2.n;
    return x;
}

void qor_text_free(qor_text *x) { free(x); }

/* embed_text_token, src/talker.rs:105-116. */
int32_t qor_embed_text_token(const qor_text *x, uint32_t token, float *out, int32_t nthreads) {
    const qtts_text_view *w = &x->w;
    if (token >= (uint32_t)w->text_embedding.k) return QTTS_ERANGE;
    const int32_t th = w->text_hidden_size, n1 = w->text_proj_fc1.n;
    float *raw = (float *)calloc((size_t)th, sizeof(float));
    float *h = (float *)calloc((size_t)n1, sizeof(float));
    if (!raw || !h) abort();
    qor_embed_lookup(&w->text_embedding, (int32_t)token, raw);
    qor_gemv(raw, &w->text_proj_fc1, h, nthreads);
    for (int32_t j = 0; j < n1; j++) h[j] += w->text_proj_fc1_bias[j];
    for (int32_t j = 0; j < n1; j++) h[j] = qor_silu(h[j]);
    qor_gemv(h, &w->text_proj_fc2, out, nthreads);
    for (int32_t j = 0; j < x->hidden; j++) out[j] += w->text_proj_fc2_bias[j];
    free(raw);
    free(h);
    return QTTS_OK;
}

static int32_t codec_row(const qor_talker *t, int32_t codec_vocab, uint32_t tok, float *out) {
    if (tok >= (uint32_t)codec_vocab) return QTTS_ERANGE;
    qor_embed_codec_token(t, tok, out);
    return QTTS_OK;
}

/* The rows prefill_custom_voice runs (src/generate_new.rs:84-177):
 *  speaker:  role x3 | codec [THINK, THINK_BOS, lang, THINK_EOS, spk, PAD] + [TTS_PAD x5, TTS_BOS]
 *            | BOS + text[0] (when there is text)
 *  voice:    role x3 | codec [THINK, THINK_BOS, lang, THINK_EOS] + TTS_PAD | voice embedding
 *            | PAD + TTS_BOS | BOS + text[0] (when there is text)
 * rows holds 10 x hidden floats; *L receives 9 or 10. */
int32_t qor_build_custom_voice_prompt(const qor_talker *t, const qor_text *x, int32_t codec_vocab,
                                      const uint32_t *tokens, int32_t n_text, uint32_t speaker_id,
                                      uint32_t language_id, const float *voice, float *rows, int32_t *L,
                                      int32_t nthreads) {
    const int32_t H = x->hidden;
    *L = 0;
    int32_t r = 0, rc = QTTS_OK;
    float *a = (float *)calloc((size_t)H, sizeof(float));
    float *b = (float *)calloc((size_t)H, sizeof(float));
    if (!a || !b) abort();
    const uint32_t role[3] = {IM_START, ASSISTANT, NEWLINE};
    for (int i = 0; i < 3 && rc == QTTS_OK; i++) rc = qor_embed_text_token(x, role[i], rows + (size_t)(r++) * H, nthreads);
    /* the TTS_PAD and TTS_BOS projections (build_tts_pad_bos, src/generate_new.rs:70-80) */
    float *pad = (float *)calloc((size_t)H, sizeof(float));
    float *bos = (float *)calloc((size_t)H, sizeof(float));
    if (!pad || !bos) abort();
    if (rc == QTTS_OK) rc = qor_embed_text_token(x, TTS_PAD, pad, nthreads);
    if (rc == QTTS_OK) rc = qor_embed_text_token(x, TTS_BOS, bos, nthreads);
    if (rc == QTTS_OK && voice) {
        const uint32_t prefix[4] = {CODEC_THINK, CODEC_THINK_BOS, language_id, CODEC_THINK_EOS};
        for (int i = 0; i < 4 && rc == QTTS_OK; i++) {
            rc = codec_row(t, codec_vocab, prefix[i], a);
            float *o = rows + (size_t)(r++) * H;
            for (int32_t j = 0; j < H && rc == QTTS_OK; j++) o[j] = a[j] + pad[j];
        }
        if (rc == QTTS_OK) memcpy(rows + (size_t)(r++) * H, voice, sizeof(float) * H);
        if (rc == QTTS_OK) {
            rc = codec_row(t, codec_vocab, CODEC_PAD, a);
            float *o = rows + (size_t)(r++) * H;
            for (int32_t j = 0; j < H && rc == QTTS_OK; j++) o[j] = a[j] + bos[j];
        }
    } else if (rc == QTTS_OK) {
        const uint32_t codec[6] = {CODEC_THINK, CODEC_THINK_BOS, language_id, CODEC_THINK_EOS, speaker_id, CODEC_PAD};
        for (int i = 0; i < 6 && rc == QTTS_OK; i++) {
            rc = codec_row(t, codec_vocab, codec[i], a);
            const float *ov = i < 5 ? pad : bos;
            float *o = rows + (size_t)(r++) * H;
            for (int32_t j = 0; j < H && rc == QTTS_OK; j++) o[j] = a[j] + ov[j];
        }
    }
    free(pad);
    free(bos);
    if (rc == QTTS_OK && n_text > 0) {
        rc = codec_row(t, codec_vocab, CODEC_BOS, a);
        if (rc == QTTS_OK) rc = qor_embed_text_token(x, tokens[0], b, nthreads);
        float *o = rows + (size_t)(r++) * H;
        for (int32_t j = 0; j < H && rc == QTTS_OK; j++) o[j] = a[j] + b[j];
    }
    free(a);
    free(b);
    if (rc == QTTS_OK) *L = r;
    return rc;
}

/* prefill_custom_voice, src/generate_new.rs:84-188: the prompt rows through
 * prefill_talker_raw, then the codec head; *position = the rows run (9 or 10,
 * src/generate_new.rs:216). */
int32_t qor_prefill_custom_voice(const qor_talker *t, const qor_text *x, int32_t codec_vocab, const uint32_t *tokens,
                                 int32_t n_text, uint32_t speaker_id, uint32_t language_id, const float *voice,
                                 qor_kv *kv, float *last_hidden, float *logits, int32_t *position, int32_t nthreads) {
    float *rows = (float *)calloc((size_t)10 * x->hidden, sizeof(float));
    if (!rows) abort();
    int32_t L = 0;
    int32_t rc = qor_build_custom_voice_prompt(t, x, codec_vocab, tokens, n_text, speaker_id, language_id, voice, rows,
                                               &L, nthreads);
    if (rc == QTTS_OK) rc = qor_prefill_talker_raw(t, rows, L, kv, last_hidden, nthreads);
    if (rc == QTTS_OK) qor_apply_codec_head(t, last_hidden, logits, nthreads);
    if (rc == QTTS_OK) *position = L;
    free(rows);
    return rc;
}

/* build_trailing_text, src/generate_new.rs:314-326: text_proj(tokens[1..])
 * then TTS_EOS; out holds max(n_text, 1) rows. */
int32_t qor_build_trailing_text(const qor_text *x, const uint32_t *tokens, int32_t n_text, float *out, int32_t *rows,
                                int32_t nthreads) {
    int32_t r = 0, rc = QTTS_OK;
    *rows = 0;
    for (int32_t i = 1; i < n_text && rc == QTTS_OK; i++)
        rc = qor_embed_text_token(x, tokens[i], out + (size_t)(r++) * x->hidden, nthreads);
    if (rc == QTTS_OK) rc = qor_embed_text_token(x, TTS_EOS, out + (size_t)(r++) * x->hidden, nthreads);
    if (rc == QTTS_OK) *rows = r;
    return rc;
}

/* generate_speech from token ids to codes, src/generate_new.rs:191-300:
 * prefill_custom_voice, build_trailing_text, the TTS_PAD row, the frame loop. */
int32_t qor_generate_speech_codes(const qor_talker *t, const qor_predictor *p, const qor_text *x, int32_t codec_vocab,
                                  const uint32_t *tokens, int32_t n_text, uint32_t speaker_id, uint32_t language_id,
                                  const float *voice, qor_kv *talker_kv, qor_kv *predictor_kv,
                                  const qtts_loop_params *params, uint64_t seed, uint32_t *codes, int32_t *n_frames,
                                  int32_t nthreads) {
    const int32_t H = x->hidden;
    float *last_hidden = (float *)calloc((size_t)H, sizeof(float));
    float *logits = (float *)calloc((size_t)codec_vocab, sizeof(float));
    float *trailing = (float *)calloc((size_t)(n_text > 1 ? n_text : 1) * H, sizeof(float));
    float *pad = (float *)calloc((size_t)H, sizeof(float));
    if (!last_hidden || !logits || !trailing || !pad) abort();
    int32_t position = 0, rows = 0;
    *n_frames = 0;
    int32_t rc = qor_prefill_custom_voice(t, x, codec_vocab, tokens, n_text, speaker_id, language_id, voice, talker_kv,
                                          last_hidden, logits, &position, nthreads);
    if (rc == QTTS_OK) rc = qor_build_trailing_text(x, tokens, n_text, trailing, &rows, nthreads);
    if (rc == QTTS_OK) rc = qor_embed_text_token(x, TTS_PAD, pad, nthreads);
    if (rc == QTTS_OK)
        rc = qor_generate_codes(t, p, talker_kv, predictor_kv, last_hidden, logits, position, trailing, rows, pad,
                                params, seed, codes, n_frames, nthreads);
    free(last_hidden);
    free(logits);
    free(trailing);
    free(pad);
    return rc;
}

/* prefill_talker, src/talker.rs:467-488: row i is embed_text_token(tokens[i])
 * when is_text[i] is nonzero, else embed_codec_token(tokens[i]); the rows in
 * sequence order then go through prefill_talker_raw (src/talker.rs:364-462),
 * which leaves the final-normed last row in last_hidden.  x may be NULL when
 * no row is text. */
int32_t qor_prefill_talker(const qor_talker *t, const qor_text *x, const uint32_t *tokens, const int32_t *is_text,
                           int32_t seq_len, qor_kv *kv, float *last_hidden, int32_t nthreads) {
    if (seq_len < 1) return QTTS_EINVAL;
    const int32_t hid = qor_talker_hidden(t);
    float *rows = (float *)calloc((size_t)seq_len * hid, sizeof(float));
    if (!rows) abort();
    int32_t rc = QTTS_OK;
    for (int32_t i = 0; i < seq_len && rc == QTTS_OK; i++) {
        float *row = rows + (size_t)i * hid;
        if (is_text[i]) {
            rc = x ? qor_embed_text_token(x, tokens[i], row, nthreads) : QTTS_ESTATE;
        } else if (tokens[i] >= (uint32_t)qor_talker_codec_rows(t)) {
            rc = QTTS_ERANGE;
        } else {
            qor_embed_codec_token(t, tokens[i], row);
        }
    }
    if (rc == QTTS_OK) rc = qor_prefill_talker_raw(t, rows, seq_len, kv, last_hidden, nthreads);
    free(rows);
    return rc;
}

/* forward_talker_decode, src/talker.rs:161-258: embed_text_token (is_text)
 * or embed_codec_token, then forward_with_embedding's step; the final-normed
 * hidden state (the first hidden values forward_with_embedding returns). */
int32_t qor_forward_talker_decode(const qor_talker *t, const qor_text *x, uint32_t token, int32_t is_text,
                                  qor_kv *kv, int32_t position, float *hidden, int32_t nthreads) {
    if (is_text && !x) return QTTS_EINVAL;
    const int32_t hid = qor_talker_hidden(t), vocab = qor_talker_vocab(t);
    float *emb = (float *)calloc((size_t)hid, sizeof(float));
    float *out = (float *)calloc((size_t)hid + vocab, sizeof(float));
    if (!emb || !out) abort();
    int32_t rc = QTTS_OK;
    if (is_text) {
        rc = qor_embed_text_token(x, token, emb, nthreads);
    } else if (token >= (uint32_t)qor_talker_codec_rows(t)) {
        rc = QTTS_ERANGE;
    } else {
        qor_embed_codec_token(t, token, emb);
    }
    if (rc == QTTS_OK) rc = qor_forward_with_embedding(t, emb, kv, position, out, nthreads);
    if (rc == QTTS_OK) memcpy(hidden, out, sizeof(float) * hid);
    free(emb);
    free(out);
    return rc;
}
