// fuzz_model_file.cpp -- a CPU fuzz pass of the .qora-tts reader
// (qtts_model_file_open, csrc/model_file.cpp; load_model, src/save.rs:262-298),
// built with AddressSanitizer and UndefinedBehaviorSanitizer by
// tests/sanitize.mk.
//
//   fuzz_model_file <file> <iterations> <seed> <scratch path>
//
// Starting from a well-formed file, each iteration writes a mutant to the
// scratch path and opens it:
//   - a cut at a random length;
//   - a structural field rewritten: an 8-byte window whose value lies in
//     1 .. file size (the u64 counts, k and n of the arrays and weights) or a
//     4-byte window whose value lies in 1 .. 100000 (the u32 header fields),
//     set to 0, 1, the value +-1, twice or half the value, the file size or
//     a huge value;
//   - random bytes flipped;
//   - two of the above.
// A mutant the reader accepts is read back in full: every array a view hands
// out, at the length the library's upload functions read it (qtts_talker_upload,
// qtts_predictor_upload, qtts_talker_text_upload, qtts_decoder_upload), so a
// view that promises more than the reader holds is an out-of-bounds read the
// sanitizers report.  A rejected mutant must carry a message.  The first
// sanitizer report ends the run with a non-zero status; a clean run prints
// the counts and exits 0.
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <random>
#include <vector>

#include "../include/qtts_file.h"

namespace {

volatile uint64_t g_sink = 0;

void touch(const void *p, size_t bytes) {
    if (!p || bytes == 0) return;
    const unsigned char *b = static_cast<const unsigned char *>(p);
    uint64_t s = 0;
    for (size_t i = 0; i < bytes; i++) s += b[i];
    g_sink = g_sink + s;
}

void touch_q4(const qtts_q4_view &w) {
    if (w.k <= 0 || w.n <= 0) return;
    touch(w.packed, (size_t)w.k * (size_t)w.n / 2);
    touch(w.scales, (size_t)w.k * (size_t)(w.n / 32) * 2);
}

void touch_layer(const qtts_layer_view &L, int hidden, int head_dim) {
    touch_q4(L.q_proj);
    touch_q4(L.k_proj);
    touch_q4(L.v_proj);
    touch_q4(L.o_proj);
    touch_q4(L.gate_proj);
    touch_q4(L.up_proj);
    touch_q4(L.down_proj);
    touch(L.q_norm, (size_t)head_dim * 2);
    touch(L.k_norm, (size_t)head_dim * 2);
    touch(L.input_norm_gamma, (size_t)hidden * 2);
    touch(L.post_attn_norm_gamma, (size_t)hidden * 2);
}

size_t pos(int v) { return v > 0 ? (size_t)v : 0; }

void touch_conv(const qtts_conv_view &v, bool depthwise) {
    const size_t wn = depthwise ? pos(v.out_channels) * pos(v.kernel_size)
                                : pos(v.in_channels) * pos(v.out_channels) * pos(v.kernel_size);
    touch(v.weight, wn * 4);
    touch(v.bias, pos(v.out_channels) * 4);
}

void touch_decoder(const qtts_decoder_view &v) {
    const size_t cd = pos(v.codebook_dim), vq = pos(v.vq_dim), hid = pos(v.hidden_size);
    const size_t ad = pos(v.num_heads) * pos(v.head_dim), inter = pos(v.intermediate_size);
    const size_t lat = pos(v.pre_conv.out_channels), cbn = pos(v.codebook_size) * cd;
    touch(v.first_codebook, cbn * 4);
    touch(v.first_output_proj, cd * vq * 4);
    touch(v.rest_output_proj, cd * vq * 4);
    for (int g = 0; g < v.num_rest && v.rest_codebooks; g++) touch(v.rest_codebooks[g], cbn * 4);
    touch_conv(v.pre_conv, false);
    touch(v.tf_input_w, lat * hid * 4);
    touch(v.tf_input_b, hid * 4);
    touch(v.tf_norm, hid * 4);
    touch(v.tf_output_w, hid * lat * 4);
    touch(v.tf_output_b, lat * 4);
    for (int l = 0; l < v.num_layers && v.layers; l++) {
        const qtts_dec_layer_view &L = v.layers[l];
        touch(L.q_proj, hid * ad * 4);
        touch(L.k_proj, hid * ad * 4);
        touch(L.v_proj, hid * ad * 4);
        touch(L.o_proj, ad * hid * 4);
        touch(L.gate_proj, hid * inter * 4);
        touch(L.up_proj, hid * inter * 4);
        touch(L.down_proj, inter * hid * 4);
        touch(L.input_norm, hid * 4);
        touch(L.post_attn_norm, hid * 4);
        touch(L.attn_scale, hid * 4);
        touch(L.mlp_scale, hid * 4);
    }
    for (int i = 0; i < v.num_upsample && v.upsample; i++) {
        const qtts_upsample_view &U = v.upsample[i];
        const size_t ch = pos(U.channels), in = pos(U.inner_dim);
        touch_conv(U.conv_t, false);
        touch_conv(U.dw_conv, true);
        touch(U.norm_w, ch * 4);
        touch(U.norm_b, ch * 4);
        touch(U.pw1_w, ch * in * 4);
        touch(U.pw1_b, in * 4);
        touch(U.pw2_w, in * ch * 4);
        touch(U.pw2_b, ch * 4);
        touch(U.gamma, ch * 4);
    }
    touch_conv(v.vocos_init, false);
    size_t ch = pos(v.vocos_init.out_channels);
    for (int b = 0; b < v.num_vocos_blocks && v.vocos_blocks; b++) {
        const qtts_vocos_block_view &B = v.vocos_blocks[b];
        touch(B.pre_snake_alpha, ch * 4);
        touch(B.pre_snake_beta, ch * 4);
        touch_conv(B.upsample, false);
        ch = pos(B.upsample.out_channels);
        for (int r = 0; r < B.num_residuals && B.residuals; r++) {
            const qtts_vocos_residual_view &R = B.residuals[r];
            touch(R.act1_alpha, ch * 4);
            touch(R.act1_beta, ch * 4);
            touch(R.act2_alpha, ch * 4);
            touch(R.act2_beta, ch * 4);
            touch_conv(R.conv1, false);
            touch_conv(R.conv2, false);
        }
    }
    touch(v.final_snake_alpha, pos(v.output_conv.in_channels) * 4);
    touch(v.final_snake_beta, pos(v.output_conv.in_channels) * 4);
    touch_conv(v.output_conv, false);
    touch(v.rope_cos, pos(v.rope_rows) * (size_t)(pos(v.head_dim) / 2) * 4);
    touch(v.rope_sin, pos(v.rope_rows) * (size_t)(pos(v.head_dim) / 2) * 4);
}

void touch_all(const qtts_model_file *f) {
    if (const qtts_talker_view *t = qtts_model_file_talker(f)) {
        for (int l = 0; l < t->num_layers && t->layers; l++) touch_layer(t->layers[l], t->hidden_size, t->head_dim);
        touch_q4(t->codec_embedding);
        touch_q4(t->codec_head);
        touch(t->final_norm_gamma, pos(t->hidden_size) * 2);
        const size_t rope = pos(t->max_position) * (size_t)(pos(t->head_dim) / 2) * 4;
        touch(t->rope_cos, rope);
        touch(t->rope_sin, rope);
    }
    if (const qtts_predictor_view *p = qtts_model_file_predictor(f)) {
        touch_q4(p->input_proj);
        if (p->input_proj.k > 0) touch(p->input_proj_bias, pos(p->input_proj.n) * 4);
        for (int g = 0; g < p->num_groups; g++) {
            if (p->codec_embeddings) touch_q4(p->codec_embeddings[g]);
            if (p->lm_heads) touch_q4(p->lm_heads[g]);
        }
        for (int l = 0; l < p->num_layers && p->layers; l++) touch_layer(p->layers[l], p->hidden_size, p->head_dim);
        touch(p->final_norm_gamma, pos(p->hidden_size) * 2);
        const size_t rope = pos(p->max_position) * (size_t)(pos(p->head_dim) / 2) * 4;
        touch(p->rope_cos, rope);
        touch(p->rope_sin, rope);
    }
    if (const qtts_text_view *x = qtts_model_file_text(f)) {
        touch_q4(x->text_embedding);
        touch_q4(x->text_proj_fc1);
        touch(x->text_proj_fc1_bias, pos(x->text_proj_fc1.n) * 4);
        touch_q4(x->text_proj_fc2);
        touch(x->text_proj_fc2_bias, pos(x->text_proj_fc2.n) * 4);
    }
    if (const qtts_decoder_view *d = qtts_model_file_decoder(f)) touch_decoder(*d);
    (void)qtts_model_file_info(f);
}

uint64_t get(const std::vector<unsigned char> &b, size_t off, int bytes) {
    uint64_t v = 0;
    for (int i = 0; i < bytes; i++) v |= (uint64_t)b[off + i] << (8 * i);
    return v;
}

void put(std::vector<unsigned char> &b, size_t off, int bytes, uint64_t v) {
    for (int i = 0; i < bytes; i++) b[off + i] = (unsigned char)(v >> (8 * i));
}

}  // namespace

int main(int argc, char **argv) {
    if (argc != 5) {
        std::fprintf(stderr, "usage: %s <file> <iterations> <seed> <scratch path>\n", argv[0]);
        return 2;
    }
    std::vector<unsigned char> base;
    if (FILE *in = std::fopen(argv[1], "rb")) {
        unsigned char buf[1 << 16];
        size_t n;
        while ((n = std::fread(buf, 1, sizeof(buf), in)) > 0) base.insert(base.end(), buf, buf + n);
        std::fclose(in);
    }
    if (base.size() < 16) {
        std::fprintf(stderr, "cannot read %s\n", argv[1]);
        return 2;
    }
    const long iters = std::atol(argv[2]);
    std::mt19937_64 rng(std::strtoull(argv[3], nullptr, 10));
    const char *scratch = argv[4];
    const uint64_t size = base.size();
    // the structural fields of the well-formed file
    std::vector<size_t> f64, f32;
    for (size_t o = 0; o + 8 <= base.size(); o++) {
        const uint64_t v = get(base, o, 8);
        if (v >= 1 && v <= size) f64.push_back(o);
    }
    for (size_t o = 0; o + 4 <= base.size(); o++) {
        const uint64_t v = get(base, o, 4);
        if (v >= 1 && v <= 100000) f32.push_back(o);
    }
    // the well-formed file itself opens and reads back
    {
        qtts_model_file *f = nullptr;
        if (qtts_model_file_open(argv[1], &f) != QTTS_OK) {
            std::fprintf(stderr, "the base file does not open: %s\n", qtts_model_file_error());
            return 1;
        }
        touch_all(f);
        qtts_model_file_close(f);
    }
    long accepted = 0, rejected = 0;
    const bool trace = std::getenv("FUZZ_TRACE") != nullptr;  // each iteration to stderr
    auto mutate = [&](std::vector<unsigned char> &m) {
        const int kind = (int)(rng() % 4);
        if (kind == 0 && m.size() > 1) {
            m.resize((size_t)(rng() % m.size()));
        } else if (kind == 1 && !f64.empty()) {
            const size_t o = f64[rng() % f64.size()];
            if (o + 8 > m.size()) return;
            const uint64_t v = get(m, o, 8);
            const uint64_t choices[] = {0, 1, v - 1, v + 1, 2 * v, v / 2, size, size - o, 1ull << 31, 1ull << 40,
                                        ~0ull, ~0ull >> 1};
            put(m, o, 8, choices[rng() % (sizeof(choices) / sizeof(choices[0]))]);
        } else if (kind == 2 && !f32.empty()) {
            const size_t o = f32[rng() % f32.size()];
            if (o + 4 > m.size()) return;
            const uint64_t v = get(m, o, 4);
            const uint64_t choices[] = {0, 1, 2, 3, v - 1, v + 1, 2 * v, v / 2, 0x7FFFFFFFull, 0xFFFFFFFFull, 0x80000000ull};
            put(m, o, 4, choices[rng() % (sizeof(choices) / sizeof(choices[0]))] & 0xFFFFFFFFull);
        } else if (!m.empty()) {
            const int flips = 1 + (int)(rng() % 4);
            for (int i = 0; i < flips; i++) m[rng() % m.size()] ^= (unsigned char)(1u << (rng() % 8));
        }
    };
    for (long it = 0; it < iters; it++) {
        std::vector<unsigned char> m = base;
        mutate(m);
        if (rng() % 4 == 0) mutate(m);
        FILE *out = std::fopen(scratch, "wb");
        if (!out) {
            std::fprintf(stderr, "cannot write %s\n", scratch);
            return 2;
        }
        if (!m.empty()) std::fwrite(m.data(), 1, m.size(), out);
        std::fclose(out);
        if (trace) std::fprintf(stderr, "iteration %ld: %zu bytes\n", it, m.size());
        qtts_model_file *f = nullptr;
        const qtts_status st = qtts_model_file_open(scratch, &f);
        if (st == QTTS_OK) {
            touch_all(f);
            qtts_model_file_close(f);
            accepted++;
        } else {
            const char *msg = qtts_model_file_error();
            if (!msg || !*msg) {
                std::fprintf(stderr, "iteration %ld: status %d without a message\n", it, (int)st);
                return 1;
            }
            rejected++;
        }
    }
    std::printf("fuzz_model_file: %ld mutants, %ld accepted and read back, %ld rejected; %zu u64 and %zu u32 "
                "fields\n",
                iters, accepted, rejected, f64.size(), f32.size());
    return 0;
}
