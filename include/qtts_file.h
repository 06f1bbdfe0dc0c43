/* qtts_file.h — reader of .qora-tts model files.
 *
 * The file is the reference's own weight container, written by save_model
 * (src/save.rs:23-46) and read by load_model (src/save.rs:262-298):
 *
 *   "QTTS" | u32 version (1) | u8 format (1 = Q4 weights, 0 = f16 weights)
 *   | talker section | code predictor section | speech decoder section
 *   | optional speaker encoder section
 *
 * all little-endian, every array as u64 element count + raw elements, every
 * Q4 weight as u64 k, u64 n, u64-counted packed bytes [k][n/2] and u64-counted
 * binary16 scales [k][n/32] (write_weight_io, src/gemv.rs:558-575).
 *
 * qtts_model_file_open reads the talker, predictor and speech decoder
 * sections into host memory and hands them out as the views
 * qtts_talker_upload, qtts_predictor_upload (include/qtts.h) and
 * qtts_decoder_upload (include/qtts_decoder.h) take, with the file's RoPE
 * tables.  All views stay valid until qtts_model_file_close.
 */
#ifndef QTTS_FILE_H
#define QTTS_FILE_H

#include <stdint.h>

#include "qtts.h"
#include "qtts_decoder.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct qtts_model_file qtts_model_file;

/* Header fields and section layout. */
typedef struct qtts_file_info {
    uint32_t version;      /* 1 */
    uint32_t format_id;    /* 1: Q4 weights */
    int32_t talker_num_kv_groups, predictor_num_kv_groups;
    int32_t mrope_sections; /* entries of mrope_section (3) */
    int32_t mrope_section[8];
    int32_t predictor_has_input_proj;
    /* speech decoder configuration (src/save.rs:170-176) */
    int32_t decoder_hidden_size, decoder_num_heads, decoder_head_dim, decoder_intermediate_size;
    int32_t decoder_sliding_window, decoder_codebook_dim;
    int32_t decoder_rest_codebooks, decoder_layers, decoder_upsample_stages, decoder_vocos_blocks;
    /* byte offsets of the sections; trailing_bytes = what follows the
     * decoder (the optional speaker encoder) */
    int64_t talker_offset, predictor_offset, decoder_offset, decoder_end, file_bytes, trailing_bytes;
} qtts_file_info;

/* load_model, src/save.rs:262-298.  Errors: QTTS_EINVAL for a missing or
 * unreadable file, a wrong magic or version, an unknown format byte or a
 * truncated or inconsistent section; QTTS_ESHAPE for a well-formed file this
 * library cannot run (format 0, f16 weights; or predictor heads and codec
 * embeddings of different counts); QTTS_ENOMEM.  The message of the last
 * failed open on this thread is qtts_model_file_error(). */
qtts_status qtts_model_file_open(const char *path, qtts_model_file **out);
const char *qtts_model_file_error(void);
void qtts_model_file_close(qtts_model_file *f);

const qtts_talker_view *qtts_model_file_talker(const qtts_model_file *f);
const qtts_predictor_view *qtts_model_file_predictor(const qtts_model_file *f);
const qtts_text_view *qtts_model_file_text(const qtts_model_file *f);
const qtts_file_info *qtts_model_file_info(const qtts_model_file *f);
const qtts_decoder_view *qtts_model_file_decoder(const qtts_model_file *f);

#ifdef __cplusplus
}
#endif

#endif /* QTTS_FILE_H */
