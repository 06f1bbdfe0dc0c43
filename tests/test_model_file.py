"""CPU tests of the .qora-tts reader (load_model, src/save.rs:262-298): a
file written in save_model's layout reads back bit for bit; the oracle gives
identical results from the file's views and from the weights it was written
from; malformed files (wrong magic, version or format byte, truncation at
any point, inconsistent lengths) are rejected with a status and a message."""
import os

import numpy as np
import pytest

import qtts
from oracle import oracle
from qtts_file_writer import TextWeights, write_model
from shapes import TINY_PREDICTOR, TINY_TALKER

PRED_ROPE_ROWS = 64  # past the 17 positions a frame uses


@pytest.fixture(scope="module")
def model():
    tw = qtts.TalkerWeights(41, TINY_TALKER)
    pw = qtts.CodePredictorWeights(41, TINY_PREDICTOR, talker_hidden=TINY_TALKER.hidden)
    text = TextWeights(41, text_vocab=96, text_hidden=64, hidden=TINY_TALKER.hidden)
    trope = oracle.build_rope_table(TINY_TALKER.head_dim, TINY_TALKER.max_position, TINY_TALKER.rope_theta)
    prope = oracle.build_rope_table(TINY_PREDICTOR.head_dim, PRED_ROPE_ROWS, TINY_PREDICTOR.rope_theta)
    return tw, pw, text, trope, prope


def _write(tmp_path, model, name="m.qora-tts", **kw):
    tw, pw, text, trope, prope = model
    path = str(tmp_path / name)
    meta = write_model(path, tw, pw, text, trope, prope, **kw)
    return path, meta


def _arr(ptr, ctype, count):
    import ctypes as C

    return np.ctypeslib.as_array(C.cast(ptr, C.POINTER(ctype)), (count,)).copy()


def _same_q4(v, w):
    assert (v.k, v.n) == (w.k, w.n)
    got = qtts.q4_from_view(v)
    assert np.array_equal(got.packed, w.packed) and np.array_equal(got.scales, w.scales)


def _same_layer(lv, L, cfg):
    import ctypes as C

    for n in ("q_proj", "k_proj", "v_proj", "o_proj", "gate_proj", "up_proj", "down_proj"):
        _same_q4(getattr(lv, n), getattr(L, n))
    for n, size in (("q_norm", cfg.head_dim), ("k_norm", cfg.head_dim), ("input_norm_gamma", cfg.hidden),
                    ("post_attn_norm_gamma", cfg.hidden)):
        assert np.array_equal(_arr(getattr(lv, n), C.c_uint16, size), getattr(L, n))


def test_round_trip(tmp_path, model):
    import ctypes as C

    tw, pw, text, trope, prope = model
    path, meta = _write(tmp_path, model, trailing=b"speaker encoder bytes")
    f = qtts.ModelFile(path)
    tv, pv, info = f.talker.view(), f.predictor.view(), f.info
    # header and layout
    assert (info.version, info.format_id) == (1, 1)
    assert (info.talker_offset, info.predictor_offset, info.decoder_offset, info.decoder_end, info.file_bytes) == (
        meta["talker_offset"], meta["predictor_offset"], meta["decoder_offset"], meta["decoder_end"],
        meta["file_bytes"])
    assert info.trailing_bytes == len(b"speaker encoder bytes")
    assert list(info.mrope_section[: info.mrope_sections]) == [24, 20, 20]
    assert info.talker_num_kv_groups == TINY_TALKER.heads // TINY_TALKER.kv_heads
    dc = meta["decoder"].cfg
    assert (info.decoder_hidden_size, info.decoder_num_heads, info.decoder_head_dim, info.decoder_intermediate_size,
            info.decoder_sliding_window, info.decoder_codebook_dim) == (dc.hidden, dc.heads, dc.head_dim, dc.inter,
                                                                        dc.window, dc.codebook_dim)
    assert (info.decoder_layers, info.decoder_rest_codebooks, info.decoder_upsample_stages,
            info.decoder_vocos_blocks) == (dc.layers, dc.num_rest, len(dc.upsample), len(dc.vocos))
    # talker
    assert (tv.num_layers, tv.hidden_size, tv.num_heads, tv.num_kv_heads, tv.head_dim) == (
        TINY_TALKER.layers, TINY_TALKER.hidden, TINY_TALKER.heads, TINY_TALKER.kv_heads, TINY_TALKER.head_dim)
    assert tv.max_position == TINY_TALKER.max_position
    for l in range(tv.num_layers):
        _same_layer(tv.layers[l], tw.layers[l], TINY_TALKER)
    _same_q4(tv.codec_embedding, tw.codec_embedding)
    _same_q4(tv.codec_head, tw.codec_head)
    assert np.array_equal(_arr(tv.final_norm_gamma, C.c_uint16, TINY_TALKER.hidden), tw.final_norm_gamma)
    half = TINY_TALKER.head_dim // 2
    assert np.array_equal(_arr(tv.rope_cos, C.c_float, trope[0].size), trope[0].reshape(-1))
    assert np.array_equal(_arr(tv.rope_sin, C.c_float, trope[1].size), trope[1].reshape(-1))
    assert trope[0].size == TINY_TALKER.max_position * half
    # text weights
    tx = f.text
    assert tx.text_hidden_size == text.text_hidden
    _same_q4(tx.text_embedding, text.text_embedding)
    _same_q4(tx.text_proj_fc1, text.fc1)
    _same_q4(tx.text_proj_fc2, text.fc2)
    assert np.array_equal(_arr(tx.text_proj_fc1_bias, C.c_float, text.fc1_bias.size), text.fc1_bias)
    assert np.array_equal(_arr(tx.text_proj_fc2_bias, C.c_float, text.fc2_bias.size), text.fc2_bias)
    # predictor
    assert (pv.num_layers, pv.hidden_size, pv.num_groups, pv.max_position) == (
        TINY_PREDICTOR.layers, TINY_PREDICTOR.hidden, pw.num_groups, PRED_ROPE_ROWS)
    assert info.predictor_has_input_proj == 1
    _same_q4(pv.input_proj, pw.input_proj)
    assert np.array_equal(_arr(pv.input_proj_bias, C.c_float, TINY_PREDICTOR.hidden), pw.input_proj_bias)
    for g in range(pw.num_groups):
        _same_q4(pv.codec_embeddings[g], pw.codec_embeddings[g])
        _same_q4(pv.lm_heads[g], pw.lm_heads[g])
    for l in range(pv.num_layers):
        _same_layer(pv.layers[l], pw.layers[l], TINY_PREDICTOR)
    assert f.predictor.talker_hidden == TINY_TALKER.hidden and f.predictor.num_groups == pw.num_groups
    f.close()


def test_decoder_round_trip(tmp_path, model):
    """The decoder section reads back as a view of the same arrays, and the
    oracle decodes identical audio from it."""
    path, meta = _write(tmp_path, model)
    dw = meta["decoder"]
    f = qtts.ModelFile(path)
    dv = f.decoder.view()
    c = dw.cfg
    assert (dv.hidden_size, dv.num_heads, dv.head_dim, dv.intermediate_size, dv.sliding_window, dv.codebook_dim,
            dv.codebook_size, dv.vq_dim, dv.num_rest, dv.num_layers, dv.num_upsample, dv.num_vocos_blocks,
            dv.rope_rows) == (c.hidden, c.heads, c.head_dim, c.inter, c.window, c.codebook_dim, c.codebook_size,
                              c.vq_dim, c.num_rest, c.layers, len(c.upsample), len(c.vocos), c.rope_rows)
    import ctypes as C

    assert np.array_equal(_arr(dv.rest_codebooks[1], C.c_float, dw.rest_codebooks[1].size), dw.rest_codebooks[1])
    r = dv.vocos_blocks[1].residuals[2].conv1
    ref = dw.blocks[1]["residuals"][2]["conv1"]
    assert (r.in_channels, r.out_channels, r.kernel_size, r.dilation) == (
        ref["in_channels"], ref["out_channels"], ref["kernel_size"], ref["dilation"])
    assert np.array_equal(_arr(r.weight, C.c_float, ref["weight"].size), ref["weight"])
    assert dv.upsample[0].inner_dim == dw.upsample[0]["inner"]
    codes = dw.synthetic_codes(6, 12)
    assert np.array_equal(oracle.decode_to_audio(f.decoder, codes), oracle.decode_to_audio(dw, codes))


def test_oracle_from_file_matches_weights(tmp_path, model):
    """The oracle run on the file's views gives the same bits as on the
    weights the file was written from (the file's RoPE tables are the
    tables the oracle builds)."""
    tw, pw, *_ = model
    path, _ = _write(tmp_path, model)
    f = qtts.ModelFile(path)
    t_file, t_mem = oracle.Talker(f.talker), oracle.Talker(tw)
    kv_file, kv_mem = t_file.new_kv(8), t_mem.new_kv(8)
    for pos in range(3):
        emb = qtts.synth_normal_f32(42, f"mf.emb.{pos}", TINY_TALKER.hidden)
        a = t_file.forward_with_embedding(emb, kv_file, pos)
        b = t_mem.forward_with_embedding(emb, kv_mem, pos)
        assert np.array_equal(a, b)
    p_file, p_mem = oracle.CodePredictor(f.predictor), oracle.CodePredictor(pw)
    h = qtts.synth_normal_f32(42, "mf.h", TINY_TALKER.hidden)
    s = qtts.synth_normal_f32(42, "mf.s", TINY_TALKER.hidden)
    assert np.array_equal(p_file.generate_acoustic_codes(h, s, p_file.new_kv()),
                          p_mem.generate_acoustic_codes(h, s, p_mem.new_kv()))


@pytest.mark.parametrize("flag", [0, 7])
def test_predictor_without_input_projection(tmp_path, model, flag):
    """has_proj == 1 means a projection follows; any other flag, none
    (src/save.rs:366-370): the view then has k == 0 (identity) and no bias."""
    path, _ = _write(tmp_path, model, has_proj_flag=flag)
    f = qtts.ModelFile(path)
    pv = f.predictor.view()
    assert pv.input_proj.k == 0 and not pv.input_proj_bias and f.info.predictor_has_input_proj == 0
    _same_q4(pv.codec_embeddings[0], model[1].codec_embeddings[0])


def _open_status(path):
    lib = qtts.load_library()
    import ctypes as C

    h = C.c_void_p()
    rc = lib.qtts_model_file_open(os.fsencode(path), C.byref(h))
    if rc == qtts.QTTS_OK:
        lib.qtts_model_file_close(h)
    return rc, lib.qtts_model_file_error().decode()


@pytest.mark.parametrize("kw, status, words", [
    (dict(magic=b"QTTX"), qtts.QTTS_EINVAL, "magic"),
    (dict(version=2), qtts.QTTS_EINVAL, "version 2"),
    (dict(format_id=0), qtts.QTTS_ESHAPE, "f16 weights"),
    (dict(format_id=3), qtts.QTTS_EINVAL, "unknown weight format"),
])
def test_bad_headers(tmp_path, model, kw, status, words):
    path, _ = _write(tmp_path, model, **kw)
    rc, msg = _open_status(path)
    assert rc == status and words in msg, msg


def test_head_count_must_match_embeddings(tmp_path, model):
    pw = model[1]
    path, _ = _write(tmp_path, model, lm_heads=pw.lm_heads[:-1])
    rc, msg = _open_status(path)
    assert rc == qtts.QTTS_ESHAPE and "heads" in msg, msg


def test_missing_file():
    rc, msg = _open_status("/nonexistent/model.qora-tts")
    assert rc == qtts.QTTS_EINVAL and "No such file" in msg


def test_truncated_files_are_rejected(tmp_path, model):
    """Cut at the start of every section, inside each, and one byte short of
    the end of the decoder section: always EINVAL, never a crash."""
    path, meta = _write(tmp_path, model)
    data = open(path, "rb").read()
    cuts = {0, 3, 4, 8, 9, 20, meta["predictor_offset"] - 1, meta["predictor_offset"], meta["predictor_offset"] + 5,
            meta["decoder_offset"] - 1, meta["decoder_offset"], meta["decoder_offset"] + 30, meta["decoder_end"] - 1}
    rng = np.random.default_rng(3)
    cuts.update(int(c) for c in rng.integers(10, meta["decoder_end"], 24))
    for cut in sorted(cuts):
        p = tmp_path / f"cut{cut}"
        p.write_bytes(data[:cut])
        rc, msg = _open_status(str(p))
        assert rc == qtts.QTTS_EINVAL, (cut, msg)
        assert "truncated" in msg or "magic" in msg or "beyond the end" in msg, (cut, msg)
    # the whole decoder section and nothing after it is a complete file
    p = tmp_path / "exact"
    p.write_bytes(data[: meta["decoder_end"]])
    assert _open_status(str(p))[0] == qtts.QTTS_OK


def test_inconsistent_weight_lengths_are_rejected(tmp_path, model):
    """A packed array whose length is not k*n/2 (here: the first talker
    weight's length field made one larger)."""
    path, meta = _write(tmp_path, model)
    data = bytearray(open(path, "rb").read())
    # talker header: 8 u32 + 3 mrope u32, then q_proj: u64 k, u64 n, u64 packed length
    off = meta["talker_offset"] + 4 * 11 + 16
    n = int.from_bytes(data[off:off + 8], "little")
    data[off:off + 8] = (n + 1).to_bytes(8, "little")
    p = tmp_path / "badlen"
    p.write_bytes(bytes(data))
    rc, msg = _open_status(str(p))
    assert rc == qtts.QTTS_EINVAL and "packed length" in msg, msg


def test_snake_lengths_must_match_their_convolutions(tmp_path, model):
    """A SnakeBeta with fewer entries than the channels of the convolution it
    feeds (found by the sanitized fuzz pass of tests/fuzz_model_file.cpp: the
    reader accepted it and the decoder upload then read past the array)."""
    from qtts_file_writer import SMALL_DECODER

    for where in ("final", "pre", "act1"):
        dw = qtts.DecoderWeights(5, SMALL_DECODER)
        if where == "final":
            dw.final_snake_alpha = dw.final_snake_alpha[:-1]
            dw.final_snake_beta = dw.final_snake_beta[:-1]
        elif where == "pre":
            dw.blocks[0]["pre_snake_alpha"] = dw.blocks[0]["pre_snake_alpha"][:-1]
            dw.blocks[0]["pre_snake_beta"] = dw.blocks[0]["pre_snake_beta"][:-1]
        else:
            r = dw.blocks[-1]["residuals"][0]
            r["act1_alpha"], r["act1_beta"] = r["act1_alpha"][:-1], r["act1_beta"][:-1]
        path, _ = _write(tmp_path, model, name=f"snake_{where}.qora-tts", decoder=dw)
        rc, msg = _open_status(path)
        assert rc == qtts.QTTS_EINVAL and "input channels" in msg, (where, msg)


def test_structure_counts_are_bounded_by_the_file(tmp_path, model):
    """A layer count of 2^31 - 1 (found by the fuzz pass: the reader sized its
    layer list from the count before reading any layer) is refused before
    anything is allocated."""
    path, meta = _write(tmp_path, model)
    data = bytearray(open(path, "rb").read())
    for off in (meta["talker_offset"], meta["predictor_offset"]):  # num_layers, the first u32 of each section
        bad = bytearray(data)
        bad[off:off + 4] = (0x7FFFFFFF).to_bytes(4, "little")
        p = tmp_path / f"count{off}"
        p.write_bytes(bytes(bad))
        rc, msg = _open_status(str(p))
        assert rc == qtts.QTTS_EINVAL and "more items than the bytes left" in msg, msg
