/*
 * qtts.h — C-ABI of the MI355X (gfx950) implementation of QORA-TTS's per-code
 * token loop: Q4 GEMV/GEMM, the Talker decode step and prefill, the Code
 * Predictor frame, the sampler and the frame loop.
 *
 * The reference crate (qora-tts 0.1.0, pure Rust, CPU only) has no FFI; the
 * interface this library replaces is the set of public Rust functions the hot
 * path is called through.  Every entry point below names the function it
 * stands in for (file:line in the reference tree).
 *
 * Conventions
 *  - Host pointers unless the name ends in _device (device pointers, work is
 *    enqueued on the context's HIP stream and the call does not synchronise).
 *  - Weights are passed once, in the reference's own Q4 layout
 *    (src/gemv.rs:26-31, src/loader.rs:204-221): packed [k][n/2] bytes, low
 *    nibble = even output column, high nibble = odd column, stored nibble =
 *    q+8; scales [k][n/32] IEEE binary16 bits, one per 32 consecutive OUTPUT
 *    columns of one input row.  The library repacks to its own device layout.
 *  - Caller-owned output buffers; nothing aborts: every failure the reference
 *    turns into a panic comes back as a qtts_status, with a message from
 *    qtts_last_error().
 *  - One host thread per context.  Several contexts may share a device.
 */
#ifndef QTTS_H
#define QTTS_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum qtts_status {
    QTTS_OK = 0,
    QTTS_EINVAL = 1,  /* null pointer or invalid argument                        */
    QTTS_ESHAPE = 2,  /* dimensions do not match                                 */
    QTTS_ENOMEM = 3,  /* device or host allocation failed                        */
    QTTS_EDEVICE = 4, /* HIP runtime error                                       */
    QTTS_ENAN = 5,    /* NaN where the reference panics in partial_cmp().unwrap() */
    QTTS_ERANGE = 6,  /* position, token or KV capacity out of range             */
    QTTS_ESTATE = 7   /* call not valid in the current state                     */
} qtts_status;

/* ------------------------------------------------------------------------ */
/* Host views of weights in the reference layout (shared with the oracle).   */
/* ------------------------------------------------------------------------ */

/* Q4Weight, src/gemv.rs:26-31.  k = input dim, n = output dim (n % 32 == 0). */
typedef struct qtts_q4_view {
    const uint8_t *packed;   /* [k][n/2]  */
    const uint16_t *scales;  /* [k][n/32] binary16 bits */
    int32_t k;
    int32_t n;
} qtts_q4_view;

/* TalkerLayerWeights (src/talker.rs:19-31); also PredictorLayerWeights
 * (src/code_predictor.rs:14-26), which has the same fields. */
typedef struct qtts_layer_view {
    qtts_q4_view q_proj, k_proj, v_proj, o_proj, gate_proj, up_proj, down_proj;
    const uint16_t *q_norm;               /* [head_dim] binary16 */
    const uint16_t *k_norm;               /* [head_dim] binary16 */
    const uint16_t *input_norm_gamma;     /* [hidden]   binary16 */
    const uint16_t *post_attn_norm_gamma; /* [hidden]   binary16 */
} qtts_layer_view;

/* The decode-path part of TalkerWeights (src/talker.rs:33-56).  The text
 * embedding and text projection belong to prompt assembly and are not here. */
typedef struct qtts_talker_view {
    int32_t num_layers;
    const qtts_layer_view *layers;
    qtts_q4_view codec_embedding; /* [vocab][hidden] (k = vocab, n = hidden) */
    qtts_q4_view codec_head;      /* [hidden][vocab] */
    const uint16_t *final_norm_gamma;
    int32_t hidden_size;  /* 2048 */
    int32_t num_heads;    /* 16 */
    int32_t num_kv_heads; /* 8 */
    int32_t head_dim;     /* 128 */
    double rope_theta;    /* 1e6 */
    int32_t max_position; /* RoPE table length, 32768 (src/config.rs:142) */
    /* Optional [max_position][head_dim/2] cos/sin tables (a model file's,
     * src/save.rs:84-85); NULL: built from rope_theta (src/rope.rs:11-41). */
    const float *rope_cos;
    const float *rope_sin;
} qtts_talker_view;

/* CodePredictorWeights, src/code_predictor.rs:28-46. */
typedef struct qtts_predictor_view {
    qtts_q4_view input_proj;      /* [talker_hidden][hidden]; k == 0 means identity */
    const float *input_proj_bias; /* [hidden] or NULL */
    int32_t num_groups;           /* 15 */
    const qtts_q4_view *codec_embeddings; /* [num_groups], each [cp_vocab][embed_dim] */
    int32_t num_layers;           /* 5 */
    const qtts_layer_view *layers;
    const qtts_q4_view *lm_heads; /* [num_groups], each [hidden][cp_vocab] */
    const uint16_t *final_norm_gamma;
    int32_t hidden_size;  /* 1024 */
    int32_t num_heads;    /* 16 */
    int32_t num_kv_heads; /* 8 */
    int32_t head_dim;     /* 128 */
    double rope_theta;    /* 1e6 */
    int32_t max_position; /* RoPE table length, 65536 (src/loader.rs:862) */
    /* Optional [max_position][head_dim/2] cos/sin tables (a model file's,
     * src/save.rs:135-136); NULL: built from rope_theta (src/loader.rs:396-408). */
    const float *rope_cos;
    const float *rope_sin;
} qtts_predictor_view;

/* The prompt-assembly part of TalkerWeights (src/talker.rs:33-56; saved at
 * src/save.rs:76-81): the text embedding and the two-layer text projection. */
typedef struct qtts_text_view {
    qtts_q4_view text_embedding;     /* [text_vocab][text_hidden] */
    qtts_q4_view text_proj_fc1;      /* [text_hidden][fc1_out] */
    const float *text_proj_fc1_bias; /* [fc1_out] */
    qtts_q4_view text_proj_fc2;      /* [fc1_out][hidden] */
    const float *text_proj_fc2_bias; /* [hidden] */
    int32_t text_hidden_size;
} qtts_text_view;

/* sample_token parameters, src/generate_new.rs:38-45,329-391. */
typedef struct qtts_sampler {
    float temperature;        /* divides the scores unless == 1.0 */
    int32_t top_k;            /* filter when 0 < top_k < vocab */
    float repetition_penalty; /* applied when != 1.0 */
    int32_t greedy;           /* 1: argmax with the last index winning ties
                                 (src/generate.rs:51-56), after the penalty */
} qtts_sampler;

/* Frame-loop parameters (TTSParams, src/generate_new.rs:38-45). */
typedef struct qtts_loop_params {
    int32_t max_codes;
    qtts_sampler sampler;  /* code-0 sampler */
    uint32_t codec_eos_id; /* 2150 */
    int32_t stop_on_eos;   /* 1: stop at EOS as src/generate_new.rs:246-249;
                              0: run exactly max_codes frames */
    int32_t talker_only;   /* 1: no predictor; next talker input is
                              codec_embedding[code0] (src/generate.rs:225-227) */
} qtts_loop_params;

/* ------------------------------------------------------------------------ */
/* Context                                                                   */
/* ------------------------------------------------------------------------ */
typedef struct qtts_ctx qtts_ctx;
typedef struct qtts_q4 qtts_q4;
typedef struct qtts_kv qtts_kv;
typedef struct qtts_talker qtts_talker;
typedef struct qtts_predictor qtts_predictor;

/* Creates a context on HIP device `device` with its own stream. */
qtts_status qtts_ctx_create(int32_t device, qtts_ctx **out);
/* Releases the caller's handle.  Weights, caches and models made from the
 * context keep it alive until they are freed, in any order; the context must
 * not be used for new calls after this. */
void qtts_ctx_destroy(qtts_ctx *ctx);
/* Message of the last failed call on this context ("" if none). */
const char *qtts_last_error(const qtts_ctx *ctx);
/* The context's hipStream_t, for callers that enqueue their own work. */
void *qtts_ctx_stream(qtts_ctx *ctx);
qtts_status qtts_ctx_synchronize(qtts_ctx *ctx);
/* Library version string. */
const char *qtts_version(void);

/* ------------------------------------------------------------------------ */
/* Q4 weights and the GEMV/GEMM operators (src/gemv.rs)                      */
/* ------------------------------------------------------------------------ */

/* Uploads and repacks one Q4 weight.  Replaces building a Weight::Q4
 * (src/gemv.rs:33-36,136-142); the dequantized values are unchanged. */
qtts_status qtts_q4_upload(qtts_ctx *ctx, const qtts_q4_view *w, qtts_q4 **out);
void qtts_q4_free(qtts_q4 *w);
/* Device bytes held by the weight (reference: Weight::memory_bytes,
 * src/gemv.rs:45-50, which this equals). */
size_t qtts_q4_bytes(const qtts_q4 *w);

/* gemv(input, weight) -> output[n]; src/gemv.rs:148-154 -> gemv_q4 263-309. */
qtts_status qtts_gemv(qtts_ctx *ctx, const qtts_q4 *w, const float *input, float *output);
/* gemm(x, seq_len, weight) -> [seq_len][n]; src/gemv.rs:156-162 -> gemm_q4 311-375. */
qtts_status qtts_gemm(qtts_ctx *ctx, const qtts_q4 *w, const float *x, int32_t seq_len, float *output);
/* embed_lookup(weight, token_id, n) -> [n]; src/gemv.rs:164-176 -> embed_lookup_q4 377-400. */
qtts_status qtts_embed_lookup(qtts_ctx *ctx, const qtts_q4 *w, int32_t token_id, float *output);
/* Same operators on device buffers, enqueued on the context stream. */
qtts_status qtts_gemv_device(qtts_ctx *ctx, const qtts_q4 *w, const float *d_input, float *d_output);
qtts_status qtts_gemm_device(qtts_ctx *ctx, const qtts_q4 *w, const float *d_x, int32_t seq_len, float *d_output);
/* No counterpart in the reference: qtts_gemm_device for 1..4 rows that
 * allocates nothing, for callers that cannot allocate device memory (code
 * under HIP graph capture, tight serving loops).  Enqueued on `stream` (a
 * hipStream_t; NULL: the weight's context stream), no synchronisation.  Its
 * split-K partials and counters live in one module-scope device array per
 * device (1 MiB), shared by every call on that device: calls that overlap on
 * one GPU race.  QTTS_ERANGE for rows outside 1..4, K above 8192 or N above
 * 16384.  Same kernels and results as qtts_gemm_device for those shapes. */
qtts_status qtts_gemv_device_static(const qtts_q4 *w, const float *d_x, int32_t rows, float *d_output, void *stream);

/* ------------------------------------------------------------------------ */
/* KV cache (RawKvCache, src/gemv.rs:75-86)                                  */
/* ------------------------------------------------------------------------ */

/* empty_kv_cache(num_layers, num_kv_heads, head_dim) with a fixed capacity in
 * positions (the reference grows a Vec; capacity overflow is QTTS_ERANGE). */
qtts_status qtts_kv_create(qtts_ctx *ctx, int32_t num_layers, int32_t num_kv_heads, int32_t head_dim,
                           int32_t capacity, qtts_kv **out);
void qtts_kv_free(qtts_kv *kv);
/* cached_len (the reference keeps one per layer; all layers move together). */
int32_t qtts_kv_len(const qtts_kv *kv);
/* Resets cached_len to 0 (src/code_predictor.rs:227-231). */
qtts_status qtts_kv_clear(qtts_kv *kv);
/* Writes positions [0, len) of every layer from host arrays in the reference
 * layout k/v[layer][len][num_kv_heads][head_dim] and sets cached_len = len. */
qtts_status qtts_kv_load(qtts_kv *kv, const float *k, const float *v, int32_t len);
/* Reads positions [0, cached_len) of every layer back in the same layout. */
qtts_status qtts_kv_store(const qtts_kv *kv, float *k, float *v);

/* ------------------------------------------------------------------------ */
/* Talker (src/talker.rs)                                                    */
/* ------------------------------------------------------------------------ */
qtts_status qtts_talker_upload(qtts_ctx *ctx, const qtts_talker_view *w, qtts_talker **out);
void qtts_talker_free(qtts_talker *t);

/* forward_with_embedding(weights, embedding, kv, position) -> [hidden ++ logits];
 * src/talker.rs:263-360.  out holds hidden_size + vocab floats. */
qtts_status qtts_forward_with_embedding(qtts_talker *t, const float *embedding, qtts_kv *kv, int32_t position,
                                        float *out);
/* prefill_talker_raw(weights, x, seq_len, kv) -> final-normed last row;
 * src/talker.rs:364-462.  Requires an empty cache, as the reference does. */
qtts_status qtts_prefill_talker_raw(qtts_talker *t, const float *x, int32_t seq_len, qtts_kv *kv,
                                    float *last_hidden);
/* apply_codec_head(weights, hidden) -> logits; src/talker.rs:627-629. */
qtts_status qtts_apply_codec_head(qtts_talker *t, const float *hidden, float *logits);
/* embed_codec_token(weights, token) -> [hidden]; src/talker.rs:152-154. */
qtts_status qtts_embed_codec_token(qtts_talker *t, uint32_t token_id, float *out);
/* forward_talker_decode(weights, token, is_text, kv, position) -> the
 * final-normed hidden [hidden_size]; src/talker.rs:161-258 (the legacy decode
 * step).  The row fed is embed_text_token(token) when is_text (text weights
 * uploaded, else QTTS_ESTATE) and embed_codec_token(token) otherwise; a token
 * past its table is QTTS_ERANGE.  The cache gains one row. */
qtts_status qtts_forward_talker_decode(qtts_talker *t, uint32_t token_id, int32_t is_text, qtts_kv *kv,
                                       int32_t position, float *hidden);
/* prefill_talker(weights, tokens, kv) -> the final-normed last row
 * [hidden_size]; src/talker.rs:467-488.  The reference's (token, is_text)
 * pairs arrive as two arrays of seq_len entries: row i is
 * embed_text_token(tokens[i]) when is_text[i] is nonzero (text weights
 * uploaded, else QTTS_ESTATE) and embed_codec_token(tokens[i]) otherwise;
 * the rows then go through prefill_talker_raw (src/talker.rs:364-462).
 * Every id is checked before any work (QTTS_ERANGE past its table); the
 * cache must be empty and gains seq_len rows. */
qtts_status qtts_prefill_talker(qtts_talker *t, const uint32_t *tokens, const int32_t *is_text, int32_t seq_len,
                                qtts_kv *kv, float *last_hidden);

/* Prompt assembly (src/talker.rs:105-116, src/generate_new.rs:60-326).  The
 * text weights ride with the talker; every step below runs on the device.  */

/* Uploads TalkerWeights' text embedding and text projection (src/talker.rs:
 * 33-56) to the talker.  The text vocab must cover the TTS special tokens
 * (src/generate_new.rs:28-30); QTTS_ESTATE on a second upload. */
qtts_status qtts_talker_text_upload(qtts_talker *t, const qtts_text_view *w);
/* embed_text_token(weights, token) -> [hidden]; src/talker.rs:105-116:
 * fc2(silu(fc1(text_embedding[token]) + b1)) + b2. */
qtts_status qtts_embed_text_token(qtts_talker *t, uint32_t token_id, float *out);
/* The input rows prefill_custom_voice runs, src/generate_new.rs:60-177: the
 * role prefix, the codec prefix with the TTS pad/BOS overlay (the built-in
 * speaker path, voice_embedding NULL) or with the raw voice embedding row
 * (voice_embedding [hidden]), and BOS + the first text token.  rows receives
 * *seq_len (9, or 10 with text) rows of hidden floats. */
qtts_status qtts_build_custom_voice_prompt(qtts_talker *t, const uint32_t *text_tokens, int32_t n_text,
                                           uint32_t speaker_id, uint32_t language_id, const float *voice_embedding,
                                           float *rows, int32_t *seq_len);
/* prefill_custom_voice(...) -> (last_hidden, logits); src/generate_new.rs:
 * 84-188.  The cache must be empty; *position receives the next position
 * (9, or 10 with text; src/generate_new.rs:216). */
qtts_status qtts_prefill_custom_voice(qtts_talker *t, const uint32_t *text_tokens, int32_t n_text, uint32_t speaker_id,
                                      uint32_t language_id, const float *voice_embedding, qtts_kv *kv,
                                      float *last_hidden, float *logits, int32_t *position);
/* build_trailing_text(weights, tokens) -> rows; src/generate_new.rs:314-326:
 * the text projection of tokens[1..] then of TTS_EOS, *n_rows = max(n_text, 1)
 * rows of hidden floats. */
qtts_status qtts_build_trailing_text(qtts_talker *t, const uint32_t *text_tokens, int32_t n_text, float *rows,
                                     int32_t *n_rows);
/* generate_speech (src/generate_new.rs:191-300) from token ids to codes:
 * prefill_custom_voice, build_trailing_text, the TTS_PAD row and the frame
 * loop (qtts_generate_codes).  The tokenizer and the speech decoder are not
 * part of it.  codes / *n_frames as for qtts_generate_codes. */
qtts_status qtts_generate_speech_codes(qtts_talker *t, qtts_predictor *p, const uint32_t *text_tokens, int32_t n_text,
                                       uint32_t speaker_id, uint32_t language_id, const float *voice_embedding,
                                       qtts_kv *talker_kv, qtts_kv *predictor_kv, const qtts_loop_params *params,
                                       uint64_t seed, uint32_t *codes, int32_t *n_frames);

/* ------------------------------------------------------------------------ */
/* Code Predictor (src/code_predictor.rs)                                    */
/* ------------------------------------------------------------------------ */
qtts_status qtts_predictor_upload(qtts_ctx *ctx, const qtts_predictor_view *w, qtts_predictor **out);
void qtts_predictor_free(qtts_predictor *p);

/* generate_acoustic_codes(weights, talker_hidden, semantic_embed, kv) -> 15
 * codes; src/code_predictor.rs:218-273.  The cache is cleared first. */
qtts_status qtts_generate_acoustic_codes(qtts_predictor *p, const float *talker_hidden, const float *semantic_embed,
                                         qtts_kv *kv, uint32_t *codes);
/* get_acoustic_embeddings_sum(weights, codes) -> [embed_dim];
 * src/code_predictor.rs:280-293.  codes holds num_groups entries. */
qtts_status qtts_get_acoustic_embeddings_sum(qtts_predictor *p, const uint32_t *codes, float *out);
/* predict_codes(weights, talker_hidden, kv, _position) -> num_groups rows
 * of logits; src/code_predictor.rs:126-213 (the legacy single step): the
 * projected talker_hidden goes through the stack at the cache offset (RoPE
 * at that offset) and every head reads the final-normed row.  logits is
 * [num_groups][cp_vocab].  The cache is NOT cleared and gains one row;
 * QTTS_ERANGE when it is full.  Offsets at or past max_position (the
 * table's rows) skip the rotation, as src/code_predictor.rs:105-107 does. */
qtts_status qtts_predict_codes(qtts_predictor *p, const float *talker_hidden, qtts_kv *kv, float *logits);

/* ------------------------------------------------------------------------ */
/* Sampler and frame loop (src/generate_new.rs)                              */
/* ------------------------------------------------------------------------ */

/* sample_token(logits, params, prev_tokens, rng) on the device;
 * src/generate_new.rs:329-391 with simple_rand 17-22.  *rng is updated. */
qtts_status qtts_sample_token(qtts_ctx *ctx, const float *logits, int32_t vocab, const qtts_sampler *params,
                              const uint32_t *prev_tokens, int32_t n_prev, uint64_t *rng, uint32_t *token);
/* sample_top_k(logits, temperature, top_k, rng) of the legacy generator,
 * src/generate.rs:50-84, on the device: temperature <= 0 is the argmax (the
 * last index of the maximum); otherwise the top_k largest logits, sorted
 * descending (ties, which the reference leaves unspecified, by ascending
 * index), p_i = exp((l_i - l_0) / temperature) normalised and summed in
 * that order against simple_rand, falling back to the k-th.  vocab is
 * 1..4096 (QTTS_ESHAPE); top_k < 1 with temperature > 0 is QTTS_EINVAL and
 * a NaN logit QTTS_ENAN (the reference panics on both).  *rng advances
 * only when sampling. */
qtts_status qtts_sample_top_k(qtts_ctx *ctx, const float *logits, int32_t vocab, float temperature, int32_t top_k,
                              uint64_t *rng, uint32_t *token);

/* The per-frame loop of generate_speech, src/generate_new.rs:229-300, run on
 * the device from the prefill outputs (last_hidden, logits) at `position`.
 * trailing_text is [trailing_len][hidden] (build_trailing_text, 314-326),
 * tts_pad_embed is [hidden].  codes is [16][max_codes] (group-major, as
 * all_codes); *n_frames receives the number of frames produced.
 * Failures: QTTS_ERANGE before anything runs when position + max_codes passes
 * the RoPE table or the cache cannot take max_codes more rows; QTTS_ENAN when
 * a NaN reaches the code-0 sampler or a predictor argmax (where the reference
 * panics).  After a failure *n_frames is 0 and both caches keep the length
 * they had (rows past it may have been written). */
qtts_status qtts_generate_codes(qtts_talker *t, qtts_predictor *p, qtts_kv *talker_kv, qtts_kv *predictor_kv,
                                const float *last_hidden, const float *logits, int32_t position,
                                const float *trailing_text, int32_t trailing_len, const float *tts_pad_embed,
                                const qtts_loop_params *params, uint64_t seed, uint32_t *codes,
                                int32_t *n_frames);

/* `batch` independent loops of generate_speech (src/generate_new.rs:229-300)
 * in lockstep over the shared weights -- the batched long-form case.  Stream
 * b has its own prefilled talker cache talker_kvs[b] (all of one capacity),
 * last_hidden + b*hidden, logits + b*vocab, positions[b], trailing text
 * trailing_text + b*trailing_len*hidden and seeds[b]; its codes go to
 * codes + b*16*max_codes ([16][max_codes] as above) and its frame count to
 * n_frames[b].  The predictor caches are internal.  Every product runs on the
 * matrix cores with one row per stream.  QTTS_ESHAPE when a weight cannot
 * use them (a scale above 8188 in magnitude); at most 64 streams.  Failures
 * as for qtts_generate_codes: QTTS_ENAN when any stream meets a NaN, and then
 * no stream's n_frames or cache length moves. */
qtts_status qtts_generate_codes_batch(qtts_talker *t, qtts_predictor *p, int32_t batch, qtts_kv *const *talker_kvs,
                                      const float *last_hidden, const float *logits, const int32_t *positions,
                                      const float *trailing_text, int32_t trailing_len, const float *tts_pad_embed,
                                      const qtts_loop_params *params, const uint64_t *seeds, uint32_t *codes,
                                      int32_t *n_frames);

#ifdef __cplusplus
}
#endif

#endif /* QTTS_H */
