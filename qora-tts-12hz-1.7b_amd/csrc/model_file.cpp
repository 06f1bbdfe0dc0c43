// model_file.cpp — .qora-tts reader (load_model, src/save.rs:262-298).
//
// Sections are read in the order save_model writes them (src/save.rs:23-46):
// talker (load_talker, src/save.rs:300-351), code predictor (load_predictor,
// src/save.rs:353-409), speech decoder (load_decoder_weights,
// src/save.rs:447-546).  Each array is read into its own host vector, so the
// views are naturally aligned whatever the array's offset in the file.  Every
// element count is checked against the bytes left in the file before anything
// is allocated.
#include "../../include/qtts_file.h"
#include "../../include/qtts_decoder.h"

#include <cerrno>
#include <cstdio>
#include <cstring>
#include <deque>
#include <new>
#include <string>
#include <vector>

namespace {

thread_local std::string g_error;

// The fewest file bytes an item of each structure count takes (its headers
// and u64 array counts with empty arrays), so that a count can be bounded by
// the bytes left: an array 8, a Q4 weight 32 (k, n and two counts), a layer
// 7 weights and 4 norm vectors, an upsample stage its channel count, two
// convolutions (5 and 3 dimensions, weight and bias each) and 7 vectors, a
// vocos block 2 vectors, a convolution and its residual count, a residual 4
// vectors and 2 convolutions of 6 dimensions.
constexpr uint64_t kVecMinBytes = 8, kWeightMinBytes = 32;
constexpr uint64_t kLayerMinBytes = 7 * kWeightMinBytes + 4 * kVecMinBytes;
constexpr uint64_t kUpsampleMinBytes = 4 + (20 + 2 * kVecMinBytes) + (12 + 2 * kVecMinBytes) + 7 * kVecMinBytes;
constexpr uint64_t kVocosBlockMinBytes = 2 * kVecMinBytes + (20 + 2 * kVecMinBytes) + 4;
constexpr uint64_t kResidualMinBytes = 4 * kVecMinBytes + 2 * (24 + 2 * kVecMinBytes);

struct FileReader {
    FILE *f = nullptr;
    int64_t pos = 0, size = 0;
    std::string err;

    bool fail(const std::string &m) {
        if (err.empty()) err = m + " (at byte " + std::to_string(pos) + ")";
        return false;
    }
    bool bytes(void *dst, size_t n, const char *what) {
        if ((int64_t)n > size - pos) return fail(std::string("truncated file reading ") + what);
        if (n && fread(dst, 1, n, f) != n) return fail(std::string("read error in ") + what);
        pos += (int64_t)n;
        return true;
    }
    bool u8(uint8_t *v, const char *what) { return bytes(v, 1, what); }
    bool u32(uint32_t *v, const char *what) {
        uint8_t b[4];
        if (!bytes(b, 4, what)) return false;
        *v = (uint32_t)b[0] | (uint32_t)b[1] << 8 | (uint32_t)b[2] << 16 | (uint32_t)b[3] << 24;
        return true;
    }
    bool u64(uint64_t *v, const char *what) {
        uint8_t b[8];
        if (!bytes(b, 8, what)) return false;
        *v = 0;
        for (int i = 7; i >= 0; i--) *v = *v << 8 | b[i];
        return true;
    }
    // A u32 count or dimension that must fit in int32.
    bool dim(int32_t *v, const char *what) {
        uint32_t u;
        if (!u32(&u, what)) return false;
        if (u > 0x7FFFFFFFu) return fail(std::string(what) + " out of range");
        *v = (int32_t)u;
        return true;
    }
    // A structure count (layers, weights, stages): items that each take at
    // least `min_bytes` of the file, bounded by the bytes left before
    // anything is sized by it.
    bool items(int32_t *v, uint64_t min_bytes, const char *what) {
        if (!dim(v, what)) return false;
        if ((uint64_t)*v > (uint64_t)(size - pos) / min_bytes)
            return fail(std::string(what) + ": more items than the bytes left");
        return true;
    }
    // u64 element count of `elem`-byte elements, bounded by the bytes left.
    bool count(uint64_t *n, size_t elem, const char *what) {
        if (!u64(n, what)) return false;
        if (*n > (uint64_t)(size - pos) / elem) return fail(std::string(what) + ": length beyond the end of the file");
        return true;
    }
};

}  // namespace

struct qtts_model_file {
    std::deque<std::vector<uint8_t>> u8s;
    std::deque<std::vector<uint16_t>> u16s;
    std::deque<std::vector<float>> f32s;
    std::vector<qtts_layer_view> talker_layers, predictor_layers;
    std::vector<qtts_q4_view> codec_embeddings, lm_heads;
    qtts_talker_view talker{};
    qtts_predictor_view predictor{};
    qtts_text_view text{};
    qtts_file_info info{};

    // write_f16_vec_io / read_f16_vec_io (src/gemv.rs:577-583,611-619)
    bool f16_vec(FileReader &r, const uint16_t **out, uint64_t *len, const char *what) {
        if (!r.count(len, 2, what)) return false;
        u16s.emplace_back((size_t)*len);
        std::vector<uint16_t> &v = u16s.back();
        uint8_t *raw = reinterpret_cast<uint8_t *>(v.data());
        if (!r.bytes(raw, (size_t)*len * 2, what)) return false;
        for (size_t i = 0; i < v.size(); i++) v[i] = (uint16_t)(raw[2 * i] | raw[2 * i + 1] << 8);
        *out = v.data();
        return true;
    }
    // write_f32_vec_io / read_f32_vec_io (src/gemv.rs:585-591,621-629)
    bool f32_vec(FileReader &r, const float **out, uint64_t *len, const char *what) {
        if (!r.count(len, 4, what)) return false;
        f32s.emplace_back((size_t)*len);
        std::vector<float> &v = f32s.back();
        uint8_t *raw = reinterpret_cast<uint8_t *>(v.data());
        if (!r.bytes(raw, (size_t)*len * 4, what)) return false;
        for (size_t i = 0; i < v.size(); i++) {
            const uint32_t b = (uint32_t)raw[4 * i] | (uint32_t)raw[4 * i + 1] << 8 | (uint32_t)raw[4 * i + 2] << 16 |
                               (uint32_t)raw[4 * i + 3] << 24;
            std::memcpy(&v[i], &b, 4);
        }
        *out = v.data();
        return true;
    }
    // read_weight_io with format 1 (src/gemv.rs:639-650): u64 k, u64 n,
    // u64-counted packed bytes, u64-counted binary16 scales.
    bool q4(FileReader &r, qtts_q4_view *w, const std::string &name) {
        uint64_t k, n, plen, slen;
        const char *what = name.c_str();
        if (!r.u64(&k, what) || !r.u64(&n, what)) return false;
        if (k == 0 || n == 0 || n % 32 != 0 || k > 0x7FFFFFFF || n > 0x7FFFFFFF)
            return r.fail(name + ": shape " + std::to_string(k) + "x" + std::to_string(n) +
                          " (n must be a positive multiple of 32)");
        if (!r.count(&plen, 1, what)) return false;
        if (plen != k * n / 2) return r.fail(name + ": packed length " + std::to_string(plen) + " != k*n/2");
        u8s.emplace_back((size_t)plen);
        if (!r.bytes(u8s.back().data(), (size_t)plen, what)) return false;
        const uint16_t *sc;
        if (!f16_vec(r, &sc, &slen, what)) return false;
        if (slen != k * n / 32) return r.fail(name + ": scale count " + std::to_string(slen) + " != k*n/32");
        w->packed = u8s.back().data();
        w->scales = sc;
        w->k = (int32_t)k;
        w->n = (int32_t)n;
        return true;
    }
    bool gamma(FileReader &r, const uint16_t **out, uint64_t want, const std::string &name) {
        uint64_t len;
        if (!f16_vec(r, out, &len, name.c_str())) return false;
        if (want && len != want)
            return r.fail(name + ": length " + std::to_string(len) + ", expected " + std::to_string(want));
        return true;
    }
    // TalkerLayerWeights / PredictorLayerWeights field order (src/save.rs:61-72).
    bool layer(FileReader &r, qtts_layer_view *L, int32_t hidden, int32_t head_dim, const std::string &p) {
        return q4(r, &L->q_proj, p + ".q_proj") && q4(r, &L->k_proj, p + ".k_proj") &&
               q4(r, &L->v_proj, p + ".v_proj") && q4(r, &L->o_proj, p + ".o_proj") &&
               gamma(r, &L->q_norm, (uint64_t)head_dim, p + ".q_norm") &&
               gamma(r, &L->k_norm, (uint64_t)head_dim, p + ".k_norm") &&
               q4(r, &L->gate_proj, p + ".gate_proj") && q4(r, &L->up_proj, p + ".up_proj") &&
               q4(r, &L->down_proj, p + ".down_proj") &&
               gamma(r, &L->input_norm_gamma, (uint64_t)hidden, p + ".input_norm") &&
               gamma(r, &L->post_attn_norm_gamma, (uint64_t)hidden, p + ".post_attn_norm");
    }
    // The two RoPE tables of a section: equal lengths, whole rows of head_dim/2.
    bool rope(FileReader &r, int32_t head_dim, const float **cs, const float **sn, int32_t *rows, const char *what) {
        uint64_t lc, ls;
        if (!f32_vec(r, cs, &lc, what) || !f32_vec(r, sn, &ls, what)) return false;
        const uint64_t half = (uint64_t)head_dim / 2;
        if (head_dim <= 0 || head_dim % 2 || lc != ls || lc == 0 || lc % half || lc / half > 0x7FFFFFFF)
            return r.fail(std::string(what) + ": cos/sin tables of " + std::to_string(lc) + "/" + std::to_string(ls) +
                          " values for head_dim " + std::to_string(head_dim));
        *rows = (int32_t)(lc / half);
        return true;
    }

    // load_talker, src/save.rs:300-351
    bool read_talker(FileReader &r) {
        qtts_talker_view &t = talker;
        int32_t layers, text_hidden, sec;
        if (!r.items(&layers, kLayerMinBytes, "talker num_layers") || !r.dim(&t.hidden_size, "talker hidden_size") ||
            !r.dim(&text_hidden, "talker text_hidden_size") || !r.dim(&t.num_heads, "talker num_heads") ||
            !r.dim(&t.num_kv_heads, "talker num_kv_heads") || !r.dim(&t.head_dim, "talker head_dim") ||
            !r.dim(&info.talker_num_kv_groups, "talker num_kv_groups") || !r.dim(&sec, "mrope_section length"))
            return false;
        if (sec > 8) return r.fail("mrope_section longer than 8");
        info.mrope_sections = sec;
        for (int i = 0; i < sec; i++)
            if (!r.dim(&info.mrope_section[i], "mrope_section")) return false;
        talker_layers.resize((size_t)layers);
        for (int32_t l = 0; l < layers; l++)
            if (!layer(r, &talker_layers[(size_t)l], t.hidden_size, t.head_dim, "talker.layers." + std::to_string(l)))
                return false;
        uint64_t len;
        if (!q4(r, &t.codec_embedding, "talker.codec_embedding") || !q4(r, &text.text_embedding, "talker.text_embedding") ||
            !q4(r, &text.text_proj_fc1, "talker.text_proj_fc1") ||
            !f32_vec(r, &text.text_proj_fc1_bias, &len, "talker.text_proj_fc1_bias"))
            return false;
        if (len != (uint64_t)text.text_proj_fc1.n) return r.fail("talker.text_proj_fc1_bias: length mismatch");
        if (!q4(r, &text.text_proj_fc2, "talker.text_proj_fc2") ||
            !f32_vec(r, &text.text_proj_fc2_bias, &len, "talker.text_proj_fc2_bias"))
            return false;
        if (len != (uint64_t)text.text_proj_fc2.n) return r.fail("talker.text_proj_fc2_bias: length mismatch");
        if (!q4(r, &t.codec_head, "talker.codec_head") ||
            !gamma(r, &t.final_norm_gamma, (uint64_t)t.hidden_size, "talker.final_norm") ||
            !rope(r, t.head_dim, &t.rope_cos, &t.rope_sin, &t.max_position, "talker rope tables"))
            return false;
        text.text_hidden_size = text_hidden;
        t.num_layers = layers;
        t.layers = talker_layers.data();
        t.rope_theta = 0.0;  // the file's tables are used
        return true;
    }

    // load_predictor, src/save.rs:353-409
    bool read_predictor(FileReader &r) {
        qtts_predictor_view &p = predictor;
        int32_t layers, groups, heads_lm;
        uint8_t has_proj;
        if (!r.items(&layers, kLayerMinBytes, "predictor num_layers") || !r.dim(&p.hidden_size, "predictor hidden_size") ||
            !r.dim(&p.num_heads, "predictor num_heads") || !r.dim(&p.num_kv_heads, "predictor num_kv_heads") ||
            !r.dim(&p.head_dim, "predictor head_dim") ||
            !r.dim(&info.predictor_num_kv_groups, "predictor num_kv_groups") || !r.u8(&has_proj, "has_proj"))
            return false;
        // any flag other than 1 means "no projection" (src/save.rs:366-370)
        info.predictor_has_input_proj = has_proj == 1;
        if (has_proj == 1) {
            uint64_t len;
            if (!q4(r, &p.input_proj, "predictor.input_proj") ||
                !f32_vec(r, &p.input_proj_bias, &len, "predictor.input_proj_bias"))
                return false;
            if (len != (uint64_t)p.input_proj.n) return r.fail("predictor.input_proj_bias: length mismatch");
        }
        if (!r.items(&groups, kWeightMinBytes, "predictor codec embedding count")) return false;
        codec_embeddings.resize((size_t)groups);
        for (int32_t g = 0; g < groups; g++)
            if (!q4(r, &codec_embeddings[(size_t)g], "predictor.codec_embeddings." + std::to_string(g))) return false;
        predictor_layers.resize((size_t)layers);
        for (int32_t l = 0; l < layers; l++)
            if (!layer(r, &predictor_layers[(size_t)l], p.hidden_size, p.head_dim,
                       "predictor.layers." + std::to_string(l)))
                return false;
        if (!r.items(&heads_lm, kWeightMinBytes, "predictor lm head count")) return false;
        lm_heads.resize((size_t)heads_lm);
        for (int32_t g = 0; g < heads_lm; g++)
            if (!q4(r, &lm_heads[(size_t)g], "predictor.lm_heads." + std::to_string(g))) return false;
        if (!gamma(r, &p.final_norm_gamma, (uint64_t)p.hidden_size, "predictor.final_norm") ||
            !rope(r, p.head_dim, &p.rope_cos, &p.rope_sin, &p.max_position, "predictor rope tables"))
            return false;
        p.num_groups = groups;
        p.codec_embeddings = codec_embeddings.data();
        p.num_layers = layers;
        p.layers = predictor_layers.data();
        p.lm_heads = lm_heads.data();
        p.rope_theta = 0.0;
        return true;
    }

    // An f32 array of exactly `want` values (0: any length, returned in *len).
    bool vec(FileReader &r, const float **out, uint64_t want, const std::string &name, uint64_t *len = nullptr) {
        uint64_t n;
        if (!f32_vec(r, out, &n, name.c_str())) return false;
        if (want && n != want)
            return r.fail(name + ": length " + std::to_string(n) + ", expected " + std::to_string(want));
        if (len) *len = n;
        return true;
    }
    // load_conv1d (6 dims), load_conv_t1d (5), load_dw_conv (3), src/save.rs:411-445.
    bool conv(FileReader &r, qtts_conv_view *c, int kind, const std::string &name) {
        int32_t dims[6] = {0, 0, 0, 1, 0, 1};
        const int nd = kind == 0 ? 6 : (kind == 1 ? 5 : 3);
        for (int i = 0; i < nd; i++)
            if (!r.dim(&dims[i], name.c_str())) return false;
        if (kind == 2) {  // channels, kernel_size, padding
            c->in_channels = c->out_channels = dims[0];
            c->kernel_size = dims[1];
            c->padding = dims[2];
            c->stride = c->dilation = 1;
        } else {
            c->in_channels = dims[0];
            c->out_channels = dims[1];
            c->kernel_size = dims[2];
            c->stride = dims[3];
            c->padding = dims[4];
            c->dilation = kind == 0 ? dims[5] : 1;
        }
        const uint64_t wn = kind == 2 ? (uint64_t)c->out_channels * c->kernel_size
                                      : (uint64_t)c->in_channels * c->out_channels * c->kernel_size;
        return vec(r, &c->weight, wn, name + ".weight") && vec(r, &c->bias, (uint64_t)c->out_channels, name + ".bias");
    }

    std::vector<const float *> rest_codebooks;
    std::vector<qtts_dec_layer_view> dec_layers;
    std::vector<qtts_upsample_view> dec_upsample;
    std::vector<qtts_vocos_block_view> dec_blocks;
    std::deque<std::vector<qtts_vocos_residual_view>> dec_residuals;
    qtts_decoder_view decoder{};

    // load_decoder_weights, src/save.rs:447-546.
    bool read_decoder(FileReader &r) {
        qtts_file_info &d = info;
        qtts_decoder_view &w = decoder;
        if (!r.dim(&d.decoder_hidden_size, "decoder hidden_size") || !r.dim(&d.decoder_num_heads, "decoder num_heads") ||
            !r.dim(&d.decoder_head_dim, "decoder head_dim") ||
            !r.dim(&d.decoder_intermediate_size, "decoder intermediate_size") ||
            !r.dim(&d.decoder_sliding_window, "decoder sliding_window") ||
            !r.dim(&d.decoder_codebook_dim, "decoder codebook_dim"))
            return false;
        w.hidden_size = d.decoder_hidden_size;
        w.num_heads = d.decoder_num_heads;
        w.head_dim = d.decoder_head_dim;
        w.intermediate_size = d.decoder_intermediate_size;
        w.sliding_window = d.decoder_sliding_window;
        w.codebook_dim = d.decoder_codebook_dim;
        const uint64_t cd = (uint64_t)w.codebook_dim, hid = (uint64_t)w.hidden_size;
        const uint64_t ad = (uint64_t)w.num_heads * w.head_dim, inter = (uint64_t)w.intermediate_size;
        if (cd == 0 || hid == 0 || ad == 0) return r.fail("decoder: zero dimension");
        uint64_t n;
        if (!vec(r, &w.first_codebook, 0, "decoder.first_codebook", &n)) return false;
        if (n % cd) return r.fail("decoder.first_codebook: not whole rows of codebook_dim");
        w.codebook_size = (int32_t)(n / cd);
        if (!vec(r, &w.first_output_proj, 0, "decoder.first_output_proj", &n)) return false;
        if (n % cd) return r.fail("decoder.first_output_proj: not whole rows of codebook_dim");
        w.vq_dim = (int32_t)(n / cd);
        if (!r.items(&d.decoder_rest_codebooks, kVecMinBytes, "decoder codebook count")) return false;
        w.num_rest = d.decoder_rest_codebooks;
        rest_codebooks.resize((size_t)w.num_rest);
        for (int32_t g = 0; g < w.num_rest; g++)
            if (!vec(r, &rest_codebooks[(size_t)g], (uint64_t)w.codebook_size * cd,
                     "decoder.rest_codebooks." + std::to_string(g)))
                return false;
        w.rest_codebooks = rest_codebooks.data();
        if (!vec(r, &w.rest_output_proj, cd * (uint64_t)w.vq_dim, "decoder.rest_output_proj") ||
            !conv(r, &w.pre_conv, 0, "decoder.pre_conv"))
            return false;
        const uint64_t lat = (uint64_t)w.pre_conv.out_channels;
        if (!vec(r, &w.tf_input_w, lat * hid, "decoder.tf_input_w") || !vec(r, &w.tf_input_b, hid, "decoder.tf_input_b") ||
            !r.items(&d.decoder_layers, 11 * kVecMinBytes, "decoder layer count"))
            return false;
        w.num_layers = d.decoder_layers;
        dec_layers.resize((size_t)w.num_layers);
        for (int32_t l = 0; l < w.num_layers; l++) {
            qtts_dec_layer_view &L = dec_layers[(size_t)l];
            const std::string p = "decoder.layers." + std::to_string(l);
            if (!vec(r, &L.q_proj, hid * ad, p + ".q_proj") || !vec(r, &L.k_proj, hid * ad, p + ".k_proj") ||
                !vec(r, &L.v_proj, hid * ad, p + ".v_proj") || !vec(r, &L.o_proj, ad * hid, p + ".o_proj") ||
                !vec(r, &L.gate_proj, hid * inter, p + ".gate_proj") || !vec(r, &L.up_proj, hid * inter, p + ".up_proj") ||
                !vec(r, &L.down_proj, inter * hid, p + ".down_proj") || !vec(r, &L.input_norm, hid, p + ".input_norm") ||
                !vec(r, &L.post_attn_norm, hid, p + ".post_attn_norm") ||
                !vec(r, &L.attn_scale, hid, p + ".attn_scale") || !vec(r, &L.mlp_scale, hid, p + ".mlp_scale"))
                return false;
        }
        w.layers = dec_layers.data();
        if (!vec(r, &w.tf_norm, hid, "decoder.tf_norm") || !vec(r, &w.tf_output_w, hid * lat, "decoder.tf_output_w") ||
            !vec(r, &w.tf_output_b, lat, "decoder.tf_output_b") ||
            !r.items(&d.decoder_upsample_stages, kUpsampleMinBytes, "decoder upsample count"))
            return false;
        w.num_upsample = d.decoder_upsample_stages;
        dec_upsample.resize((size_t)w.num_upsample);
        for (int32_t u = 0; u < w.num_upsample; u++) {
            qtts_upsample_view &U = dec_upsample[(size_t)u];
            const std::string p = "decoder.upsample." + std::to_string(u);
            if (!r.dim(&U.channels, "upsample channels") || !conv(r, &U.conv_t, 1, p + ".conv_t") ||
                !conv(r, &U.dw_conv, 2, p + ".dw_conv"))
                return false;
            const uint64_t ch = (uint64_t)U.channels;
            uint64_t inner;
            if (!vec(r, &U.norm_w, ch, p + ".norm_w") || !vec(r, &U.norm_b, ch, p + ".norm_b") ||
                !vec(r, &U.pw1_w, 0, p + ".pw1_w", &n) || !vec(r, &U.pw1_b, 0, p + ".pw1_b", &inner))
                return false;
            if (inner == 0 || n != ch * inner) return r.fail(p + ".pw1_w: length is not channels x inner");
            U.inner_dim = (int32_t)inner;
            if (!vec(r, &U.pw2_w, inner * ch, p + ".pw2_w") || !vec(r, &U.pw2_b, ch, p + ".pw2_b") ||
                !vec(r, &U.gamma, ch, p + ".gamma"))
                return false;
        }
        w.upsample = dec_upsample.data();
        if (!conv(r, &w.vocos_init, 0, "decoder.vocos_init") || !r.items(&d.decoder_vocos_blocks, kVocosBlockMinBytes, "vocos block count"))
            return false;
        w.num_vocos_blocks = d.decoder_vocos_blocks;
        dec_blocks.resize((size_t)w.num_vocos_blocks);
        for (int32_t b = 0; b < w.num_vocos_blocks; b++) {
            qtts_vocos_block_view &B = dec_blocks[(size_t)b];
            const std::string p = "decoder.vocos." + std::to_string(b);
            uint64_t na;
            int32_t nres;
            if (!vec(r, &B.pre_snake_alpha, 0, p + ".pre_snake_alpha", &na) ||
                !vec(r, &B.pre_snake_beta, na, p + ".pre_snake_beta") || !conv(r, &B.upsample, 1, p + ".upsample") ||
                !r.items(&nres, kResidualMinBytes, "vocos residual count"))
                return false;
            // a SnakeBeta has one (alpha, beta) per channel of the
            // convolution it feeds (src/conv.rs:347-372)
            if (na != (uint64_t)B.upsample.in_channels)
                return r.fail(p + ".pre_snake_alpha: length is not the upsample's input channels");
            dec_residuals.emplace_back((size_t)nres);
            std::vector<qtts_vocos_residual_view> &res = dec_residuals.back();
            for (int32_t i = 0; i < nres; i++) {
                qtts_vocos_residual_view &R = res[(size_t)i];
                const std::string q = p + ".residuals." + std::to_string(i);
                uint64_t na2;
                if (!vec(r, &R.act1_alpha, 0, q + ".act1_alpha", &na) || !vec(r, &R.act1_beta, na, q + ".act1_beta") ||
                    !conv(r, &R.conv1, 0, q + ".conv1") || !vec(r, &R.act2_alpha, 0, q + ".act2_alpha", &na2) ||
                    !vec(r, &R.act2_beta, na2, q + ".act2_beta") || !conv(r, &R.conv2, 0, q + ".conv2"))
                    return false;
                if (na != (uint64_t)R.conv1.in_channels || na2 != (uint64_t)R.conv2.in_channels)
                    return r.fail(q + ": a SnakeBeta's length is not its convolution's input channels");
            }
            B.num_residuals = nres;
            B.residuals = res.data();
        }
        w.vocos_blocks = dec_blocks.data();
        uint64_t na, nc;
        if (!vec(r, &w.final_snake_alpha, 0, "decoder.final_snake_alpha", &na) ||
            !vec(r, &w.final_snake_beta, na, "decoder.final_snake_beta") ||
            !conv(r, &w.output_conv, 0, "decoder.output_conv") || !vec(r, &w.rope_cos, 0, "decoder.rope_cos", &nc) ||
            !vec(r, &w.rope_sin, nc, "decoder.rope_sin"))
            return false;
        if (na != (uint64_t)w.output_conv.in_channels)
            return r.fail("decoder.final_snake_alpha: length is not output_conv's input channels");
        const uint64_t half = (uint64_t)w.head_dim / 2;
        if (half == 0 || nc % half) return r.fail("decoder rope tables: not whole rows of head_dim/2");
        w.rope_rows = (int32_t)(nc / half);
        return true;
    }
};

extern "C" {

qtts_status qtts_model_file_open(const char *path, qtts_model_file **out) {
    g_error.clear();
    if (!path || !out) {
        g_error = "null argument";
        return QTTS_EINVAL;
    }
    *out = nullptr;
    FileReader r;
    r.f = fopen(path, "rb");
    if (!r.f) {
        g_error = std::string(path) + ": " + std::strerror(errno);
        return QTTS_EINVAL;
    }
    qtts_status st = QTTS_OK;
    qtts_model_file *m = nullptr;
    try {
        m = new qtts_model_file();
        if (fseeko(r.f, 0, SEEK_END) != 0 || (r.size = (int64_t)ftello(r.f)) < 0 || fseeko(r.f, 0, SEEK_SET) != 0) {
            r.fail("cannot size the file");
        } else {
            m->info.file_bytes = r.size;
            // header: magic, version, format (src/save.rs:266-277)
            char magic[4];
            uint32_t version = 0;
            uint8_t format = 0;
            if (r.bytes(magic, 4, "magic") && std::memcmp(magic, "QTTS", 4) != 0) r.fail("invalid magic (expected QTTS)");
            if (r.err.empty() && r.u32(&version, "version") && version != 1)
                r.fail("version " + std::to_string(version) + ", expected 1");
            if (r.err.empty() && r.u8(&format, "format")) {
                m->info.version = version;
                m->info.format_id = format;
                if (format == 0) {
                    r.fail("format 0 (f16 weights) is not supported: the loop runs Q4 weights");
                    st = QTTS_ESHAPE;
                } else if (format != 1) {
                    r.fail("unknown weight format " + std::to_string(format));
                }
            }
            if (r.err.empty()) {
                m->info.talker_offset = r.pos;
                if (m->read_talker(r)) {
                    m->info.predictor_offset = r.pos;
                    if (m->read_predictor(r)) {
                        m->info.decoder_offset = r.pos;
                        if (m->read_decoder(r)) {
                            m->info.decoder_end = r.pos;
                            m->info.trailing_bytes = r.size - r.pos;
                        }
                    }
                }
            }
            if (r.err.empty() && m->predictor.num_groups != (int32_t)m->lm_heads.size()) {
                r.fail("predictor has " + std::to_string(m->predictor.num_groups) + " codec embeddings and " +
                       std::to_string(m->lm_heads.size()) + " heads");
                st = QTTS_ESHAPE;
            }
        }
    } catch (const std::bad_alloc &) {
        r.err = "out of host memory";
        st = QTTS_ENOMEM;
    }
    fclose(r.f);
    if (!r.err.empty()) {
        delete m;
        g_error = std::string(path) + ": " + r.err;
        return st == QTTS_OK ? QTTS_EINVAL : st;
    }
    *out = m;
    return QTTS_OK;
}

const char *qtts_model_file_error(void) { return g_error.c_str(); }

void qtts_model_file_close(qtts_model_file *f) { delete f; }

const qtts_talker_view *qtts_model_file_talker(const qtts_model_file *f) { return f ? &f->talker : nullptr; }
const qtts_predictor_view *qtts_model_file_predictor(const qtts_model_file *f) { return f ? &f->predictor : nullptr; }
const qtts_text_view *qtts_model_file_text(const qtts_model_file *f) { return f ? &f->text : nullptr; }
const qtts_file_info *qtts_model_file_info(const qtts_model_file *f) { return f ? &f->info : nullptr; }
const qtts_decoder_view *qtts_model_file_decoder(const qtts_model_file *f) { return f ? &f->decoder : nullptr; }

}  // extern "C"
