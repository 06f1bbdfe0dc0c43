"""Writes .qora-tts model files for the reader's tests, in the byte layout of
save_model (src/save.rs:23-46): the talker section (src/save.rs:48-89), the
code predictor section (src/save.rs:91-137) and the speech decoder section
(src/save.rs:168-257), with the array encodings of src/gemv.rs:558-597
(u64 element count, then little-endian elements)."""
import struct

import numpy as np

import qtts


class _Out:
    def __init__(self):
        self.parts = []
        self.size = 0

    def raw(self, b: bytes):
        self.parts.append(b)
        self.size += len(b)

    def u8(self, v):
        self.raw(struct.pack("<B", v))

    def u32(self, v):
        self.raw(struct.pack("<I", v))

    def u64(self, v):
        self.raw(struct.pack("<Q", v))

    def f16v(self, a):  # write_f16_vec_io
        a = np.ascontiguousarray(a, dtype="<u2").reshape(-1)
        self.u64(a.size)
        self.raw(a.tobytes())

    def f32v(self, a):  # write_f32_vec_io
        a = np.ascontiguousarray(a, dtype="<f4").reshape(-1)
        self.u64(a.size)
        self.raw(a.tobytes())

    def q4(self, w: "qtts.Q4Weight"):  # write_weight_io, Weight::Q4
        self.u64(w.k)
        self.u64(w.n)
        p = np.ascontiguousarray(w.packed, dtype=np.uint8).reshape(-1)
        self.u64(p.size)
        self.raw(p.tobytes())
        self.f16v(w.scales)


class TextWeights(qtts.TextWeights):
    """Synthetic text embedding + two-layer text projection (fc1 text_hidden ->
    text_hidden, fc2 text_hidden -> hidden)."""

    def __init__(self, seed, text_vocab, text_hidden, hidden):
        super().__init__(seed, text_vocab, text_hidden, hidden)


def _layer(o, L):  # src/save.rs:61-72
    for n in ("q_proj", "k_proj", "v_proj", "o_proj"):
        o.q4(getattr(L, n))
    o.f16v(L.q_norm)
    o.f16v(L.k_norm)
    for n in ("gate_proj", "up_proj", "down_proj"):
        o.q4(getattr(L, n))
    o.f16v(L.input_norm_gamma)
    o.f16v(L.post_attn_norm_gamma)


def _conv(o, c, kind):
    """save_conv1d (kind 0), save_conv_t1d (1), save_dw_conv (2), src/save.rs:139-166."""
    if kind == 2:
        dims = (c["out_channels"], c["kernel_size"], c["padding"])
    else:
        dims = (c["in_channels"], c["out_channels"], c["kernel_size"], c["stride"], c["padding"])
        if kind == 0:
            dims += (c["dilation"],)
    for d in dims:
        o.u32(d)
    o.f32v(c["weight"])
    o.f32v(c["bias"])


def _decoder(o, dw):
    """save_decoder, src/save.rs:168-257, from a qtts.DecoderWeights."""
    c = dw.cfg
    for v in (c.hidden, c.heads, c.head_dim, c.inter, c.window, c.codebook_dim):
        o.u32(v)
    o.f32v(dw.first_codebook)
    o.f32v(dw.first_output_proj)
    o.u32(len(dw.rest_codebooks))
    for cb in dw.rest_codebooks:
        o.f32v(cb)
    o.f32v(dw.rest_output_proj)
    _conv(o, dw.pre_conv, 0)
    o.f32v(dw.tf_input_w)
    o.f32v(dw.tf_input_b)
    o.u32(len(dw.layers))
    for L in dw.layers:
        for n in ("q_proj", "k_proj", "v_proj", "o_proj", "gate_proj", "up_proj", "down_proj", "input_norm",
                  "post_attn_norm", "attn_scale", "mlp_scale"):
            o.f32v(L[n])
    o.f32v(dw.tf_norm)
    o.f32v(dw.tf_output_w)
    o.f32v(dw.tf_output_b)
    o.u32(len(dw.upsample))
    for u in dw.upsample:
        o.u32(u["conv_t"]["out_channels"])
        _conv(o, u["conv_t"], 1)
        _conv(o, u["dw_conv"], 2)
        for n in ("norm_w", "norm_b", "pw1_w", "pw1_b", "pw2_w", "pw2_b", "gamma"):
            o.f32v(u[n])
    _conv(o, dw.vocos_init, 0)
    o.u32(len(dw.blocks))
    for b in dw.blocks:
        o.f32v(b["pre_snake_alpha"])
        o.f32v(b["pre_snake_beta"])
        _conv(o, b["upsample"], 1)
        o.u32(len(b["residuals"]))
        for r in b["residuals"]:
            o.f32v(r["act1_alpha"])
            o.f32v(r["act1_beta"])
            _conv(o, r["conv1"], 0)
            o.f32v(r["act2_alpha"])
            o.f32v(r["act2_beta"])
            _conv(o, r["conv2"], 0)
    o.f32v(dw.final_snake_alpha)
    o.f32v(dw.final_snake_beta)
    _conv(o, dw.output_conv, 0)
    o.f32v(dw.rope_cos)
    o.f32v(dw.rope_sin)


# A small decoder for the reader's tests.
SMALL_DECODER = qtts.DecoderConfig(hidden=64, heads=4, head_dim=16, inter=128, window=8, codebook_dim=32,
                                   codebook_size=64, vq_dim=64, latent=128, num_rest=3, layers=2, upsample=(2,),
                                   vocos_channels=96, vocos=((96, 48, 4, 2), (48, 24, 6, 3)), rope_rows=64)


def write_model(path, tw, pw, text, talker_rope, predictor_rope, *, decoder=None, magic=b"QTTS", version=1,
                format_id=1, mrope_section=(24, 20, 20), has_proj_flag=1, trailing=b"", lm_heads=None):
    """Writes tw (TalkerWeights), pw (CodePredictorWeights) and text
    (TextWeights) with the given (cos, sin) RoPE tables, then the decoder
    (a qtts.DecoderWeights; default a small random one) and `trailing`
    bytes.  Returns the section offsets and the decoder weights."""
    o = _Out()
    o.raw(magic)
    o.u32(version)
    o.u8(format_id)
    meta = {"talker_offset": o.size}
    c = tw.cfg
    # save_talker, src/save.rs:48-89
    for v in (len(tw.layers), c.hidden, text.text_hidden, c.heads, c.kv_heads, c.head_dim, c.heads // c.kv_heads,
              len(mrope_section)):
        o.u32(v)
    for s in mrope_section:
        o.u32(s)
    for L in tw.layers:
        _layer(o, L)
    o.q4(tw.codec_embedding)
    o.q4(text.text_embedding)
    o.q4(text.fc1)
    o.f32v(text.fc1_bias)
    o.q4(text.fc2)
    o.f32v(text.fc2_bias)
    o.q4(tw.codec_head)
    o.f16v(tw.final_norm_gamma)
    o.f32v(talker_rope[0])
    o.f32v(talker_rope[1])
    # save_predictor, src/save.rs:91-137
    meta["predictor_offset"] = o.size
    p = pw.cfg
    for v in (len(pw.layers), p.hidden, p.heads, p.kv_heads, p.head_dim, p.heads // p.kv_heads):
        o.u32(v)
    o.u8(has_proj_flag)
    if has_proj_flag == 1:
        o.q4(pw.input_proj)
        o.f32v(pw.input_proj_bias)
    o.u32(len(pw.codec_embeddings))
    for e in pw.codec_embeddings:
        o.q4(e)
    for L in pw.layers:
        _layer(o, L)
    heads = pw.lm_heads if lm_heads is None else lm_heads
    o.u32(len(heads))
    for h in heads:
        o.q4(h)
    o.f16v(pw.final_norm_gamma)
    o.f32v(predictor_rope[0])
    o.f32v(predictor_rope[1])
    meta["decoder_offset"] = o.size
    dw = decoder if decoder is not None else qtts.DecoderWeights(5, SMALL_DECODER)
    _decoder(o, dw)
    meta["decoder"] = dw
    meta["decoder_end"] = o.size
    o.raw(trailing)
    meta["file_bytes"] = o.size
    with open(path, "wb") as f:
        for part in o.parts:
            f.write(part)
    return meta
