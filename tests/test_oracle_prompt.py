"""Pins the oracle's prompt assembly (oracle/qtts_oracle_prompt.c):
embed_text_token against a float64 model of src/talker.rs:105-116, and the
rows of prefill_custom_voice (src/generate_new.rs:60-177), build_trailing_text
(src/generate_new.rs:314-326) and generate_speech (src/generate_new.rs:
191-300) against compositions written here from the reference's description
out of the oracle's already-pinned pieces (embed_codec_token, the prefill,
the codec head, the frame loop).  Every composition is exact (the same f32
operations), so a dropped overlay, a wrong token, a swapped row or a wrong
position fails bit for bit."""
import numpy as np
import pytest

import numpy_model as nm
import qtts
from oracle import oracle

# a talker with the real codec vocabulary (the special codec tokens are
# 2148-2157) and a text vocabulary that covers the TTS special tokens
TALKER = qtts.StackConfig(layers=2, hidden=256, heads=4, kv_heads=2, head_dim=128, inter=512, vocab=3072,
                          max_position=4096)
PREDICTOR = qtts.StackConfig(layers=2, hidden=128, heads=2, kv_heads=1, head_dim=128, inter=256, vocab=256,
                             max_position=65536)
TEXT_HIDDEN = 64
SPEAKER, LANGUAGE = 3000, 2050
TOKENS = [9707, 11, 1879, 0, 151643, 77091, 5]


@pytest.fixture(scope="module")
def model():
    tw = qtts.TalkerWeights(81, TALKER)
    pw = qtts.CodePredictorWeights(81, PREDICTOR, talker_hidden=TALKER.hidden)
    text = qtts.TextWeights(82, qtts.TEXT_VOCAB_1P7B, TEXT_HIDDEN, TALKER.hidden)
    ot = oracle.Talker(tw, nthreads=1)
    return tw, pw, text, ot, oracle.CodePredictor(pw, nthreads=1), oracle.Text(ot, text, nthreads=1)


def f64_text(text, token):
    """embed_text_token in float64: fc2(silu(fc1(emb[token]) + b1)) + b2."""
    emb = nm.dequant(text.text_embedding)[token]
    h = emb @ nm.dequant(text.fc1) + text.fc1_bias.astype(np.float64)
    h = nm.silu(h)
    return h @ nm.dequant(text.fc2) + text.fc2_bias.astype(np.float64)


def rel(got, ref):
    got, ref = np.asarray(got, np.float64), np.asarray(ref, np.float64)
    return float(np.max(np.abs(got - ref)) / np.max(np.abs(ref)))


@pytest.mark.parametrize("token", [0, 198, 151644, qtts.TTS_PAD, qtts.TTS_EOS, qtts.TEXT_VOCAB_1P7B - 1])
def test_embed_text_token_float64(model, token):
    _, _, text, _, _, ox = model
    assert rel(ox.embed_text_token(token), f64_text(text, token)) < 1e-5


def test_embed_text_token_range(model):
    ox = model[5]
    with pytest.raises(oracle.OracleError) as e:
        ox.embed_text_token(qtts.TEXT_VOCAB_1P7B)
    assert e.value.status == qtts.QTTS_ERANGE


def _expected_rows(ot, ox, tokens, voice):
    ett, ect = ox.embed_text_token, ot.embed_codec_token
    rows = [ett(qtts.IM_START), ett(qtts.ASSISTANT), ett(qtts.NEWLINE)]
    pad, bos = ett(qtts.TTS_PAD), ett(qtts.TTS_BOS)
    if voice is not None:
        rows += [ect(t) + pad for t in (qtts.CODEC_THINK, qtts.CODEC_THINK_BOS, LANGUAGE, qtts.CODEC_THINK_EOS)]
        rows.append(np.asarray(voice, np.float32))
        rows.append(ect(qtts.CODEC_PAD) + bos)
    else:
        codec = (qtts.CODEC_THINK, qtts.CODEC_THINK_BOS, LANGUAGE, qtts.CODEC_THINK_EOS, SPEAKER, qtts.CODEC_PAD)
        rows += [ect(t) + (pad if i < 5 else bos) for i, t in enumerate(codec)]
    if len(tokens):
        rows.append(ect(qtts.CODEC_BOS) + ett(tokens[0]))
    return np.stack(rows)


@pytest.mark.parametrize("voice", [False, True], ids=["speaker", "voice"])
@pytest.mark.parametrize("tokens", [TOKENS, []], ids=["text", "no_text"])
def test_prompt_rows(model, voice, tokens):
    _, _, text, ot, _, ox = model
    v = qtts.synth_normal_f32(83, "voice", TALKER.hidden) if voice else None
    got = ox.build_custom_voice_prompt(tokens, SPEAKER, LANGUAGE, v)
    ref = _expected_rows(ot, ox, tokens, v)
    assert got.shape == ref.shape == (10 if tokens else 9, TALKER.hidden)
    assert np.array_equal(got, ref)
    # one overlay row in float64: codec_emb[THINK] + text_proj(TTS_PAD)
    cod = nm.dequant(model[0].codec_embedding)[qtts.CODEC_THINK]
    assert rel(got[3], cod + f64_text(text, qtts.TTS_PAD)) < 1e-5


@pytest.mark.parametrize("voice", [False, True], ids=["speaker", "voice"])
def test_prefill_custom_voice(model, voice):
    _, _, text, ot, _, ox = model
    v = qtts.synth_normal_f32(84, "voice", TALKER.hidden) if voice else None
    kv = ot.new_kv(32)
    lh, lg, pos = ox.prefill_custom_voice(TOKENS, SPEAKER, LANGUAGE, kv, v)
    rows = ox.build_custom_voice_prompt(TOKENS, SPEAKER, LANGUAGE, v)
    kv2 = ot.new_kv(32)
    lh2 = ot.prefill_talker_raw(rows, rows.shape[0], kv2)
    assert pos == rows.shape[0] == 10 and len(kv) == len(kv2) == 10
    assert np.array_equal(lh, lh2) and np.array_equal(lg, ot.apply_codec_head(lh2))


@pytest.mark.parametrize("tokens", [TOKENS, TOKENS[:1], []], ids=["many", "one", "none"])
def test_trailing_text(model, tokens):
    ox = model[5]
    got = ox.build_trailing_text(tokens)
    ref = np.stack([ox.embed_text_token(t) for t in list(tokens[1:]) + [qtts.TTS_EOS]])
    assert got.shape == ref.shape == (max(len(tokens), 1), TALKER.hidden)
    assert np.array_equal(got, ref)


@pytest.mark.parametrize("voice", [False, True], ids=["speaker", "voice"])
def test_generate_speech_codes_composition(model, voice):
    tw, pw, text, ot, op, ox = model
    v = qtts.synth_normal_f32(85, "voice", TALKER.hidden) if voice else None
    params = qtts.loop_params(12, stop_on_eos=False)
    got = ox.generate_speech_codes(op, TOKENS, SPEAKER, LANGUAGE, ot.new_kv(32), op.new_kv(), params, 7, v)
    kv = ot.new_kv(32)
    lh, lg, pos = ox.prefill_custom_voice(TOKENS, SPEAKER, LANGUAGE, kv, v)
    trailing = ox.build_trailing_text(TOKENS)
    pad = ox.embed_text_token(qtts.TTS_PAD)
    ref = oracle.generate_codes(ot, op, kv, op.new_kv(), lh, lg, pos, trailing, pad, params, seed=7)
    assert got.shape == ref.shape == (16, 12)
    assert np.array_equal(got, ref)


@pytest.mark.parametrize("n", [1, 6, 13])
def test_prefill_talker_composition(model, n):
    """prefill_talker (src/talker.rs:467-488): row i from embed_text_token or
    embed_codec_token by its flag, in sequence order, then prefill_talker_raw;
    bit for bit, caches included (a swapped flag or row changes the bits)."""
    tw, pw, text, ot, op, ox = model
    rng = np.random.default_rng(n)
    is_text = rng.integers(0, 2, n).astype(bool)
    is_text[0] = True
    tokens = np.where(is_text, rng.integers(0, qtts.TEXT_VOCAB_1P7B, n), rng.integers(0, TALKER.vocab, n))
    tokens = tokens.astype(np.uint32)
    kv, kv2 = ot.new_kv(16), ot.new_kv(16)
    got = oracle.prefill_talker(ot, ox, tokens, is_text, kv)
    rows = np.stack([ox.embed_text_token(t) if f else ot.embed_codec_token(t) for t, f in zip(tokens, is_text)])
    ref = ot.prefill_talker_raw(rows, n, kv2)
    assert np.array_equal(got, ref) and len(kv) == len(kv2) == n
    (a, b), (c, d) = kv.store(), kv2.store()
    assert np.array_equal(a, c) and np.array_equal(b, d)
    if n > 1:  # the flags matter: all-codec rows of the same ids differ
        assert not np.array_equal(oracle.prefill_talker(ot, None, tokens % TALKER.vocab, np.zeros(n, bool),
                                                        ot.new_kv(16)), got)


def test_prefill_talker_errors(model):
    _, _, _, ot, _, ox = model
    kv = ot.new_kv(8)
    cases = (([TALKER.vocab], [False], qtts.QTTS_ERANGE), ([qtts.TEXT_VOCAB_1P7B], [True], qtts.QTTS_ERANGE),
             ([], [], qtts.QTTS_EINVAL))
    for toks, flags, status in cases:
        with pytest.raises(oracle.OracleError) as e:
            oracle.prefill_talker(ot, ox, toks, flags, kv)
        assert e.value.status == status and len(kv) == 0
    with pytest.raises(oracle.OracleError) as e:  # a text row and no text weights
        oracle.prefill_talker(ot, None, [5, 9707], [False, True], kv)
    assert e.value.status == qtts.QTTS_ESTATE and len(kv) == 0
    oracle.prefill_talker(ot, None, [5, 2148], [False, False], kv)
    assert len(kv) == 2


def test_codec_token_range(model):
    _, _, _, ot, _, ox = model
    with pytest.raises(oracle.OracleError) as e:
        ox.build_custom_voice_prompt(TOKENS, TALKER.vocab, LANGUAGE)
    assert e.value.status == qtts.QTTS_ERANGE
