/* qtts_decoder.h — the speech decoder: 16 x T codes -> 24 kHz audio.
 *
 * decode_to_audio (src/decoder.rs:394-509) on the device: codebook lookup
 * and projection, causal pre-conv, the sliding-window transformer, the
 * ConvNeXt upsample stages and the Vocos blocks (SnakeBeta, transposed and
 * causal convolutions), all in f32 like the reference.
 */
#ifndef QTTS_DECODER_H
#define QTTS_DECODER_H

#include <stdint.h>

#include "qtts.h"

#ifdef __cplusplus
extern "C" {
#endif

/* Conv1dWeight (src/conv.rs:29-38): weight [out][in][kernel].
 * ConvTranspose1dWeight (src/conv.rs:186-194): weight [in][out][kernel].
 * DepthwiseConv1dWeight (src/conv.rs:270-276): weight [channels][kernel],
 * in_channels = out_channels = channels. */
typedef struct qtts_conv_view {
    const float *weight;
    const float *bias; /* [out_channels] */
    int32_t in_channels, out_channels, kernel_size, stride, padding, dilation;
} qtts_conv_view;

/* DecoderTfLayer, src/decoder.rs:67-79; projections as [in][out]. */
typedef struct qtts_dec_layer_view {
    const float *q_proj, *k_proj, *v_proj; /* [hidden][heads*head_dim] */
    const float *o_proj;                   /* [heads*head_dim][hidden] */
    const float *gate_proj, *up_proj;      /* [hidden][intermediate] */
    const float *down_proj;                /* [intermediate][hidden] */
    const float *input_norm, *post_attn_norm, *attn_scale, *mlp_scale; /* [hidden] */
} qtts_dec_layer_view;

/* UpsampleStage, src/decoder.rs:81-92. */
typedef struct qtts_upsample_view {
    int32_t channels;
    int32_t inner_dim;          /* pw1 width (4 x channels) */
    qtts_conv_view conv_t;      /* transposed, channels -> channels */
    qtts_conv_view dw_conv;     /* depthwise, causal */
    const float *norm_w, *norm_b; /* [channels] LayerNorm */
    const float *pw1_w, *pw1_b;   /* [channels][inner], [inner] */
    const float *pw2_w, *pw2_b;   /* [inner][channels], [channels] */
    const float *gamma;           /* [channels] */
} qtts_upsample_view;

/* VocosResidual, src/decoder.rs:101-108. */
typedef struct qtts_vocos_residual_view {
    const float *act1_alpha, *act1_beta; /* [channels] */
    qtts_conv_view conv1;                /* causal, kernel 7 */
    const float *act2_alpha, *act2_beta;
    qtts_conv_view conv2;                /* kernel 1 */
} qtts_vocos_residual_view;

/* VocosBlock, src/decoder.rs:94-99. */
typedef struct qtts_vocos_block_view {
    const float *pre_snake_alpha, *pre_snake_beta; /* [upsample.in_channels] */
    qtts_conv_view upsample;                       /* transposed */
    int32_t num_residuals;
    const qtts_vocos_residual_view *residuals;
} qtts_vocos_block_view;

/* SpeechDecoderWeights, src/decoder.rs:22-65. */
typedef struct qtts_decoder_view {
    int32_t hidden_size;       /* 512 */
    int32_t num_heads;         /* 16 */
    int32_t head_dim;          /* 64 */
    int32_t intermediate_size; /* 1024 */
    int32_t sliding_window;    /* 72 */
    int32_t codebook_dim;      /* 256 */
    int32_t codebook_size;     /* entries per codebook, 2048 */
    int32_t vq_dim;            /* output projection width, 512 */
    const float *first_codebook;    /* [codebook_size][codebook_dim] */
    const float *first_output_proj; /* [codebook_dim][vq_dim] */
    int32_t num_rest;               /* 15 */
    const float *const *rest_codebooks; /* num_rest x [codebook_size][codebook_dim] */
    const float *rest_output_proj;  /* [codebook_dim][vq_dim] */
    qtts_conv_view pre_conv;        /* causal, vq_dim -> latent (1024) */
    const float *tf_input_w, *tf_input_b;   /* [latent][hidden], [hidden] */
    int32_t num_layers;
    const qtts_dec_layer_view *layers;
    const float *tf_norm;                   /* [hidden] */
    const float *tf_output_w, *tf_output_b; /* [hidden][latent], [latent] */
    int32_t num_upsample;
    const qtts_upsample_view *upsample;
    qtts_conv_view vocos_init;              /* causal, latent -> 1536 */
    int32_t num_vocos_blocks;
    const qtts_vocos_block_view *vocos_blocks;
    const float *final_snake_alpha, *final_snake_beta; /* [output_conv.in_channels] */
    qtts_conv_view output_conv;             /* causal, -> 1 channel */
    const float *rope_cos, *rope_sin;       /* [rope_rows][head_dim/2] */
    int32_t rope_rows;
} qtts_decoder_view;

typedef struct qtts_decoder qtts_decoder;

/* Copies the decoder weights to the device.  QTTS_ESHAPE for dimensions the
 * reference's pipeline cannot chain (e.g. a transposed convolution with
 * padding or a kernel not a multiple of its stride). */
qtts_status qtts_decoder_upload(qtts_ctx *ctx, const qtts_decoder_view *w, qtts_decoder **out);
void qtts_decoder_free(qtts_decoder *d);

/* Samples decode_to_audio returns for `frames` frames (0 for 0 frames). */
int64_t qtts_decoder_num_samples(const qtts_decoder *d, int32_t frames);

/* decode_to_audio, src/decoder.rs:394-509.  codes[g * ld + t] is codebook
 * g's index at frame t, g < num_rest + 1, t < frames; audio receives
 * qtts_decoder_num_samples(d, frames) samples (QTTS_ERANGE if capacity is
 * smaller, or for a code >= codebook_size).  Host buffers; the _device form
 * takes device buffers, does not synchronise and does not read the codes on
 * the host: a code >= codebook_size there reads codebook row 0. */
qtts_status qtts_decode_to_audio(qtts_decoder *d, const uint32_t *codes, int32_t frames, int32_t ld, float *audio,
                                 int64_t capacity, int64_t *n_samples);
qtts_status qtts_decode_to_audio_device(qtts_decoder *d, const uint32_t *d_codes, int32_t frames, int32_t ld,
                                        float *d_audio, int64_t capacity, int64_t *n_samples);

/* generate_speech (src/generate_new.rs:191-311) from token ids to audio:
 * qtts_generate_speech_codes's steps, then decode_to_audio of the codes
 * where the frame loop leaves them in device memory (they never cross to the
 * host).  The tokenizer is not part of it.  audio (host) receives *n_samples
 * = qtts_decoder_num_samples(d, *n_frames) floats; capacity must cover
 * qtts_decoder_num_samples(d, params->max_codes), checked before any work
 * (QTTS_ERANGE).  A generated code >= the decoder's codebook_size, where the
 * reference's lookup would panic, is QTTS_ERANGE.  The decoder must be on
 * the talker's device (QTTS_EINVAL) and read at most 16 code groups
 * (QTTS_ESHAPE).  Caches and seed as for qtts_generate_speech_codes. */
qtts_status qtts_generate_speech(qtts_talker *t, qtts_predictor *p, qtts_decoder *d, const uint32_t *text_tokens,
                                 int32_t n_text, uint32_t speaker_id, uint32_t language_id,
                                 const float *voice_embedding, qtts_kv *talker_kv, qtts_kv *predictor_kv,
                                 const qtts_loop_params *params, uint64_t seed, float *audio, int64_t capacity,
                                 int64_t *n_samples, int32_t *n_frames);

#ifdef __cplusplus
}
#endif

#endif /* QTTS_DECODER_H */
