"""Writes .qora-tts model files for the reader's tests, in the byte layout of
save_model (src/save.rs:23-46): the talker section (src/save.rs:48-89), the
code predictor section (src/save.rs:91-137) and the speech decoder section
(src/save.rs:168-257), with the array encodings of src/gemv.rs:558-597
(u64 element count, then little-endian elements).  The decoder tensors are
small random arrays: the reader only walks that section."""
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


class TextWeights:
    """Synthetic text embedding + two-layer text projection."""

    def __init__(self, seed, text_vocab, text_hidden, hidden):
        self.text_hidden = text_hidden
        self.text_embedding = qtts.Q4Weight.synthetic(seed, "text.embedding", text_vocab, text_hidden)
        self.fc1 = qtts.Q4Weight.synthetic(seed, "text.fc1", text_hidden, text_hidden)
        self.fc1_bias = qtts.synth_normal_f32(seed, "text.fc1_bias", text_hidden, 0.0, 0.02)
        self.fc2 = qtts.Q4Weight.synthetic(seed, "text.fc2", text_hidden, hidden)
        self.fc2_bias = qtts.synth_normal_f32(seed, "text.fc2_bias", hidden, 0.0, 0.02)


def _layer(o, L):  # src/save.rs:61-72
    for n in ("q_proj", "k_proj", "v_proj", "o_proj"):
        o.q4(getattr(L, n))
    o.f16v(L.q_norm)
    o.f16v(L.k_norm)
    for n in ("gate_proj", "up_proj", "down_proj"):
        o.q4(getattr(L, n))
    o.f16v(L.input_norm_gamma)
    o.f16v(L.post_attn_norm_gamma)


def _conv(o, rng, dims, wlen, blen):
    for d in dims:
        o.u32(d)
    o.f32v(rng.standard_normal(wlen).astype(np.float32))
    o.f32v(rng.standard_normal(blen).astype(np.float32))


def _decoder(o, rng, layers=2, rest=3, upsample=2, blocks=2, residuals=2):
    """A small speech decoder section in the order of src/save.rs:168-257."""
    vec = lambda n: o.f32v(rng.standard_normal(n).astype(np.float32))
    cfg = dict(hidden=64, heads=2, head_dim=32, inter=128, window=72, cb_dim=16)
    for v in cfg.values():
        o.u32(v)
    vec(32 * 16)  # first_codebook
    vec(16 * 64)  # first_output_proj
    o.u32(rest)
    for _ in range(rest):
        vec(32 * 16)
    vec(16 * 64)  # rest_output_proj
    _conv(o, rng, (64, 64, 3, 1, 1, 1), 64 * 64 * 3, 64)  # pre_conv
    vec(64 * 64)
    vec(64)
    o.u32(layers)
    for _ in range(layers):
        for n in (64 * 64,) * 4 + (64 * 128,) * 3 + (64,) * 4:
            vec(n)
    vec(64)
    vec(64 * 64)
    vec(64)
    o.u32(upsample)
    for _ in range(upsample):
        o.u32(64)
        _conv(o, rng, (64, 64, 2, 2, 0), 64 * 64 * 2, 64)  # conv_t
        _conv(o, rng, (64, 7, 3), 64 * 7, 64)  # dw_conv
        for n in (64, 64, 64 * 256, 256, 256 * 64, 64, 64):
            vec(n)
    _conv(o, rng, (64, 96, 7, 1, 3, 1), 64 * 96 * 7, 96)  # vocos_init
    o.u32(blocks)
    for _ in range(blocks):
        vec(96)
        vec(96)
        _conv(o, rng, (96, 48, 4, 2, 1), 96 * 48 * 4, 48)
        o.u32(residuals)
        for _ in range(residuals):
            vec(48)
            vec(48)
            _conv(o, rng, (48, 48, 7, 1, 3, 1), 48 * 48 * 7, 48)
            vec(48)
            vec(48)
            _conv(o, rng, (48, 48, 1, 1, 0, 1), 48 * 48, 48)
    vec(48)
    vec(48)
    _conv(o, rng, (48, 1, 7, 1, 3, 1), 48 * 7, 1)
    vec(100 * 16)  # rope tables
    vec(100 * 16)
    return dict(cfg, layers=layers, rest=rest, upsample=upsample, blocks=blocks)


def write_model(path, tw, pw, text, talker_rope, predictor_rope, *, magic=b"QTTS", version=1, format_id=1,
                mrope_section=(24, 20, 20), has_proj_flag=1, trailing=b"", lm_heads=None):
    """Writes tw (TalkerWeights), pw (CodePredictorWeights) and text
    (TextWeights) with the given (cos, sin) RoPE tables, then a synthetic
    decoder section and `trailing` bytes.  Returns the section offsets and
    the decoder configuration."""
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
    meta["decoder"] = _decoder(o, np.random.default_rng(5))
    meta["decoder_end"] = o.size
    o.raw(trailing)
    meta["file_bytes"] = o.size
    with open(path, "wb") as f:
        for part in o.parts:
            f.write(part)
    return meta
