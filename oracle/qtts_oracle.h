/*
 * qtts_oracle.h — CPU restatement of the reference's per-code loop.
 *
 * TEST INFRASTRUCTURE ONLY.  This is what the parity tests compare the HIP
 * library against, and the CPU baseline bench.py times.  Nothing in
 * the product library links, loads or calls it.
 *
 * It restates the arithmetic ORDER of the reference Rust crate (qora-tts
 * 0.1.0): the LUT GEMV with its k*n >= 4e6 split-K thread fan-out, sequential
 * f32 sums, glibc expf/sqrtf, RoPE tables built in double and cast to float.
 * Built with -O3 -ffp-contract=off (no -march), as rustc would compile the
 * crate for the default x86-64 target: no FMA contraction, no reassociation.
 */
#ifndef QTTS_ORACLE_H
#define QTTS_ORACLE_H

#include <stdint.h>

#include "../include/qtts.h"
#include "../include/qtts_decoder.h"

#ifdef __cplusplus
extern "C" {
#endif

/* std::thread::available_parallelism(): affinity mask, capped by a cgroup
 * CPU quota when one is set. */
int32_t qor_available_parallelism(void);

float qor_f16_to_f32(uint16_t h);

/* --- src/gemv.rs ---------------------------------------------------------- */
/* gemv_q4, src/gemv.rs:263-309.  nthreads = the value available_parallelism()
 * would return (<= 0: detect); it only matters when k*n >= 4e6. */
void qor_gemv(const float *input, const qtts_q4_view *w, float *out, int32_t nthreads);
/* gemm_q4, src/gemv.rs:311-375 (row results do not depend on nthreads). */
void qor_gemm(const float *x, int32_t seq_len, const qtts_q4_view *w, float *out, int32_t nthreads);
/* embed_lookup_q4, src/gemv.rs:377-400. */
void qor_embed_lookup(const qtts_q4_view *w, int32_t token_id, float *out);
/* rms_norm_f16, src/gemv.rs:406-417. */
void qor_rms_norm_f16(const float *x, const uint16_t *gamma, int32_t n, float *out);
/* softmax_raw, src/gemv.rs:433-445. */
void qor_softmax_raw(float *scores, int32_t n);
/* silu, src/gemv.rs:447-451. */
float qor_silu(float x);
/* apply_qk_norm, src/talker.rs:86-99 (= src/code_predictor.rs:84-93). */
void qor_qk_norm(float *data, int32_t num_heads, int32_t head_dim, const uint16_t *gamma);

/* --- src/rope.rs ---------------------------------------------------------- */
/* build_mrope_tables, src/rope.rs:11-41 (sections are contiguous, so this is
 * also the predictor table of src/loader.rs:859-874). */
void qor_build_rope_table(int32_t head_dim, int32_t max_pos, double theta, float *cos_table, float *sin_table);
/* Split-half rotation at one position: apply_mrope_interleaved with
 * position_ids = [p,p,p] (src/rope.rs:50-93) and apply_rope_split
 * (src/code_predictor.rs:97-121). */
void qor_rope_split(float *data, int32_t num_heads, int32_t head_dim, int32_t pos, const float *cos_table,
                    const float *sin_table);

/* --- KV cache: RawKvCache, src/gemv.rs:75-86 (token-major f32) ----------- */
typedef struct qor_kv qor_kv;
qor_kv *qor_kv_new(int32_t num_layers, int32_t num_kv_heads, int32_t head_dim, int32_t capacity);
void qor_kv_free(qor_kv *kv);
int32_t qor_kv_len(const qor_kv *kv);
void qor_kv_clear(qor_kv *kv);
/* k/v are [layer][len][kv_heads][head_dim]. */
int32_t qor_kv_load(qor_kv *kv, const float *k, const float *v, int32_t len);
int32_t qor_kv_store(const qor_kv *kv, float *k, float *v);

/* --- src/talker.rs -------------------------------------------------------- */
typedef struct qor_talker qor_talker;
/* Keeps a copy of the view (the arrays it points to must outlive it) and
 * builds the RoPE table, as load_talker does (src/loader.rs:768-775). */
qor_talker *qor_talker_new(const qtts_talker_view *w);
void qor_talker_free(qor_talker *t);
/* hidden_size, codec vocab and codec embedding rows of the talker. */
int32_t qor_talker_hidden(const qor_talker *t);
int32_t qor_talker_vocab(const qor_talker *t);
int32_t qor_talker_codec_rows(const qor_talker *t);
/* forward_with_embedding, src/talker.rs:263-360.  out = [hidden ++ logits]. */
int32_t qor_forward_with_embedding(const qor_talker *t, const float *embedding, qor_kv *kv, int32_t position,
                                   float *out, int32_t nthreads);
/* prefill_talker_raw, src/talker.rs:364-462. */
int32_t qor_prefill_talker_raw(const qor_talker *t, const float *x, int32_t seq_len, qor_kv *kv,
                               float *last_hidden, int32_t nthreads);
/* apply_codec_head, src/talker.rs:627-629. */
void qor_apply_codec_head(const qor_talker *t, const float *hidden, float *logits, int32_t nthreads);
/* embed_codec_token, src/talker.rs:152-154. */
void qor_embed_codec_token(const qor_talker *t, uint32_t token_id, float *out);

/* --- src/code_predictor.rs ----------------------------------------------- */
typedef struct qor_predictor qor_predictor;
typedef struct qor_text qor_text;
qor_predictor *qor_predictor_new(const qtts_predictor_view *w);
void qor_predictor_free(qor_predictor *p);
/* generate_acoustic_codes, src/code_predictor.rs:218-273. */
int32_t qor_generate_acoustic_codes(const qor_predictor *p, const float *talker_hidden, const float *semantic_embed,
                                    qor_kv *kv, uint32_t *codes, int32_t nthreads);
/* get_acoustic_embeddings_sum, src/code_predictor.rs:280-293. */
void qor_get_acoustic_embeddings_sum(const qor_predictor *p, const uint32_t *codes, float *out);

/* --- src/generate_new.rs ------------------------------------------------- */
/* simple_rand, src/generate_new.rs:17-22. */
float qor_simple_rand(uint64_t *state);
/* sample_argmax, src/code_predictor.rs:328-334: last index wins ties.
 * Returns QTTS_ENAN where the reference panics. */
int32_t qor_argmax(const float *logits, int32_t n, uint32_t *out);
/* sample_token, src/generate_new.rs:329-391 (greedy: argmax after penalty). */
int32_t qor_sample_token(const float *logits, int32_t vocab, const qtts_sampler *params, const uint32_t *prev_tokens,
                         int32_t n_prev, uint64_t *rng, uint32_t *token);
/* The frame loop of generate_speech, src/generate_new.rs:229-300. */
int32_t qor_generate_codes(const qor_talker *t, const qor_predictor *p, qor_kv *talker_kv, qor_kv *predictor_kv,
                           const float *last_hidden, const float *logits, int32_t position,
                           const float *trailing_text, int32_t trailing_len, const float *tts_pad_embed,
                           const qtts_loop_params *params, uint64_t seed, uint32_t *codes, int32_t *n_frames,
                           int32_t nthreads);

/* --- src/decoder.rs, src/conv.rs (qtts_oracle_decoder.c) ---------------- */
/* Samples decode_to_audio returns for `frames` frames. */
int64_t qor_decoder_num_samples(const qtts_decoder_view *w, int32_t frames);
/* decode_to_audio, src/decoder.rs:394-509; codes[g * ld + t].  QTTS_ERANGE
 * for a code past the codebook or too small an output buffer. */
int32_t qor_decode_to_audio(const qtts_decoder_view *w, const uint32_t *codes, int32_t frames, int32_t ld,
                            float *audio, int64_t capacity, int64_t *n_samples, int32_t nthreads);
/* generate::sample_top_k, src/generate.rs:50-84 (equal logits by index). */
int32_t qor_sample_top_k(const float *logits, int32_t vocab, float temperature, int32_t top_k, uint64_t *rng,
                         uint32_t *token);
/* predict_codes, src/code_predictor.rs:126-213: one step of talker_hidden
 * through the predictor at the cache offset, then all num_groups heads on the
 * final-normed row: logits [num_groups][vocab]. */
int32_t qor_predict_codes(const qor_predictor *p, const float *talker_hidden, qor_kv *kv, float *logits,
                          int32_t nthreads);
/* forward_talker_decode, src/talker.rs:161-258: the final-normed hidden of
 * one step fed embed_text_token (is_text) or embed_codec_token. */
int32_t qor_forward_talker_decode(const qor_talker *t, const qor_text *x, uint32_t token, int32_t is_text,
                                  qor_kv *kv, int32_t position, float *hidden, int32_t nthreads);
/* prefill_talker, src/talker.rs:467-488: (token, is_text) rows through
 * prefill_talker_raw.  x may be NULL when no row is text. */
int32_t qor_prefill_talker(const qor_talker *t, const qor_text *x, const uint32_t *tokens, const int32_t *is_text,
                           int32_t seq_len, qor_kv *kv, float *last_hidden, int32_t nthreads);

/* --- prompt assembly (qtts_oracle_prompt.c) ------------------------------ */
/* The text embedding and projection of TalkerWeights (src/talker.rs:33-56). */
qor_text *qor_text_new(const qtts_text_view *w);
void qor_text_free(qor_text *x);
/* embed_text_token, src/talker.rs:105-116.  QTTS_ERANGE past the text vocab. */
int32_t qor_embed_text_token(const qor_text *x, uint32_t token, float *out, int32_t nthreads);
/* The prompt rows of prefill_custom_voice (src/generate_new.rs:60-177):
 * rows [10][hidden], *L = 9 or 10; voice NULL for the built-in speaker path. */
int32_t qor_build_custom_voice_prompt(const qor_talker *t, const qor_text *x, int32_t codec_vocab,
                                      const uint32_t *tokens, int32_t n_text, uint32_t speaker_id,
                                      uint32_t language_id, const float *voice, float *rows, int32_t *L,
                                      int32_t nthreads);
/* prefill_custom_voice, src/generate_new.rs:84-188. */
int32_t qor_prefill_custom_voice(const qor_talker *t, const qor_text *x, int32_t codec_vocab, const uint32_t *tokens,
                                 int32_t n_text, uint32_t speaker_id, uint32_t language_id, const float *voice,
                                 qor_kv *kv, float *last_hidden, float *logits, int32_t *position, int32_t nthreads);
/* build_trailing_text, src/generate_new.rs:314-326: out [max(n_text,1)][hidden]. */
int32_t qor_build_trailing_text(const qor_text *x, const uint32_t *tokens, int32_t n_text, float *out, int32_t *rows,
                                int32_t nthreads);
/* generate_speech from token ids to codes, src/generate_new.rs:191-300. */
int32_t qor_generate_speech_codes(const qor_talker *t, const qor_predictor *p, const qor_text *x, int32_t codec_vocab,
                                  const uint32_t *tokens, int32_t n_text, uint32_t speaker_id, uint32_t language_id,
                                  const float *voice, qor_kv *talker_kv, qor_kv *predictor_kv,
                                  const qtts_loop_params *params, uint64_t seed, uint32_t *codes, int32_t *n_frames,
                                  int32_t nthreads);

/* Test hooks: the decoder's primitives (qtts_oracle_decoder.c), for CPU
 * checks against closed forms and float64 brute force. */
void qor_dec_causal_conv(const float *in, int32_t len, const qtts_conv_view *w, float *out, int32_t nt);
int32_t qor_dec_transposed_conv(const float *in, int32_t len, const qtts_conv_view *w, float *out, int32_t nt);
void qor_dec_depthwise_conv(const float *in, int32_t len, const qtts_conv_view *w, float *out, int32_t nt);
void qor_dec_snake(const float *in, int32_t ch, int32_t len, const float *alpha, const float *beta, float *out,
                   int32_t nt);
float qor_dec_gelu(float x);
void qor_dec_layer_norm_cf(const float *in, const float *g, const float *b, int32_t ch, int32_t len, float eps,
                           float *out);
void qor_dec_rms_norm(const float *x, const float *gamma, float eps, int32_t n, float *out);
void qor_dec_rope(float *data, int32_t heads, int32_t hd, int32_t pos, const float *cs, const float *sn,
                  int32_t rows);
void qor_dec_window_attention(const float *q, const float *k, const float *v, int32_t T, int32_t heads, int32_t hd,
                              int32_t window, float *out);
void qor_dec_codebook_lookup(const qtts_decoder_view *w, const uint32_t *codes, int32_t T, int32_t ld, float *out);

#ifdef __cplusplus
}
#endif

#endif /* QTTS_ORACLE_H */
