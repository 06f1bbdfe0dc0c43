"""GPU parity of the prompt assembly on the device against the oracle:
embed_text_token (src/talker.rs:105-116), the rows of prefill_custom_voice
(src/generate_new.rs:60-177, built-in speaker and voice-embedding paths),
the prefill itself (src/generate_new.rs:84-188), build_trailing_text
(src/generate_new.rs:314-326), and generate_speech from token ids to codes
(src/generate_new.rs:191-300) with no embedding math on the host,
prefill_talker from (token, is_text) rows (src/talker.rs:467-488) and
generate_speech from token ids to audio (src/generate_new.rs:191-311): a small
model with the real codec and text vocabularies, and the 1.7B talker and
predictor with the 1.7B text projection.

Bars: rows, hidden states and logits within 1e-3 relative (the text
projection's GEMV sums in another order than the oracle's); codes identical."""
import ctypes as C
import dataclasses

import numpy as np
import pytest

import qtts
from oracle import oracle
from shapes import FULL_PREDICTOR, FULL_TALKER, rel_err, within

pytestmark = pytest.mark.gpu

TALKER = qtts.StackConfig(layers=2, hidden=256, heads=4, kv_heads=2, head_dim=128, inter=512, vocab=3072,
                          max_position=4096)
PREDICTOR = qtts.StackConfig(layers=2, hidden=128, heads=2, kv_heads=1, head_dim=128, inter=256, vocab=256,
                             max_position=65536)
SPEAKER, LANGUAGE = 3000, 2050
TOKENS = [9707, 11, 1879, 0, 151643, 77091, 5, 1000, 20000, 151935]
TOL = 1e-3


@pytest.fixture(scope="module")
def small(ctx):
    tw = qtts.TalkerWeights(91, TALKER)
    pw = qtts.CodePredictorWeights(91, PREDICTOR, talker_hidden=TALKER.hidden)
    text = qtts.TextWeights(92, qtts.TEXT_VOCAB_1P7B, 64, TALKER.hidden)
    t, p = qtts.Talker(ctx, tw), qtts.CodePredictor(ctx, pw)
    t.attach_text(text)
    ot, op = oracle.Talker(tw, nthreads=1), oracle.CodePredictor(pw, nthreads=1)
    return t, p, ot, op, oracle.Text(ot, text, nthreads=1)


def test_text_rows(small):
    t, p, ot, op, ox = small
    for tok in (0, 198, qtts.IM_START, qtts.TTS_PAD, qtts.TTS_BOS, qtts.TTS_EOS, qtts.TEXT_VOCAB_1P7B - 1):
        assert rel_err(t.embed_text_token(tok), ox.embed_text_token(tok)) < 1e-5, tok
    for toks in (TOKENS, TOKENS[:1], []):
        got, ref = t.build_trailing_text(toks), ox.build_trailing_text(toks)
        assert got.shape == ref.shape == (max(len(toks), 1), TALKER.hidden)
        assert rel_err(got, ref) < 1e-5


@pytest.mark.parametrize("voice", [False, True], ids=["speaker", "voice"])
@pytest.mark.parametrize("tokens", [TOKENS, []], ids=["text", "no_text"])
def test_prompt_rows_and_prefill(small, voice, tokens):
    t, p, ot, op, ox = small
    v = qtts.synth_normal_f32(93, "voice", TALKER.hidden) if voice else None
    got = t.build_custom_voice_prompt(tokens, SPEAKER, LANGUAGE, v)
    ref = ox.build_custom_voice_prompt(tokens, SPEAKER, LANGUAGE, v)
    assert got.shape == ref.shape
    assert rel_err(got, ref) < 1e-5
    if voice:
        assert np.array_equal(got[7], v)  # the voice row goes in as it is
    kv, okv = t.new_kv(40), ot.new_kv(40)
    lh, lg, pos = t.prefill_custom_voice(tokens, SPEAKER, LANGUAGE, kv, v)
    olh, olg, opos = ox.prefill_custom_voice(tokens, SPEAKER, LANGUAGE, okv, v)
    assert pos == opos == ref.shape[0] and len(kv) == len(okv) == pos
    assert within(lh, olh) and within(lg, olg)
    (gk, gv), (rk, rv) = kv.store(), okv.store()
    assert within(gk, rk) and within(gv, rv)


@pytest.mark.parametrize("voice", [False, True], ids=["speaker", "voice"])
@pytest.mark.parametrize("greedy", [True, False], ids=["greedy", "sampled"])
def test_generate_speech_codes_small(small, voice, greedy):
    t, p, ot, op, ox = small
    v = qtts.synth_normal_f32(94, "voice", TALKER.hidden) if voice else None
    params = qtts.loop_params(24, greedy=greedy, stop_on_eos=False)
    got = qtts.generate_speech_codes(t, p, TOKENS, SPEAKER, LANGUAGE, t.new_kv(40), p.new_kv(), params, seed=11,
                                     voice_embedding=v)
    ref = ox.generate_speech_codes(op, TOKENS, SPEAKER, LANGUAGE, ot.new_kv(40), op.new_kv(), params, 11, v)
    assert got.shape == ref.shape == (16, 24)
    assert np.array_equal(got, ref), np.argwhere(got != ref)[:5]


def test_prompt_errors(small):
    t, p, ot, op, ox = small
    kv = t.new_kv(40)
    with pytest.raises(qtts.QttsError) as e:
        t.prefill_custom_voice([qtts.TEXT_VOCAB_1P7B], SPEAKER, LANGUAGE, kv)
    assert e.value.status == qtts.QTTS_ERANGE
    with pytest.raises(qtts.QttsError) as e:
        t.prefill_custom_voice(TOKENS, TALKER.vocab, LANGUAGE, kv)
    assert e.value.status == qtts.QTTS_ERANGE
    assert len(kv) == 0
    t.prefill_custom_voice(TOKENS, SPEAKER, LANGUAGE, kv)
    with pytest.raises(qtts.QttsError) as e:  # the cache is no longer empty
        t.prefill_custom_voice(TOKENS, SPEAKER, LANGUAGE, kv)
    assert e.value.status == qtts.QTTS_ESTATE


def _token_rows(seed, n):
    rng = np.random.default_rng(seed)
    is_text = rng.integers(0, 2, n).astype(bool)
    tokens = np.where(is_text, rng.integers(0, qtts.TEXT_VOCAB_1P7B, n), rng.integers(0, TALKER.vocab, n))
    return tokens.astype(np.uint32), is_text


@pytest.mark.parametrize("n", [1, 7, 40])
def test_prefill_talker(small, n):
    """prefill_talker (src/talker.rs:467-488) from (token, is_text) rows: the
    last hidden and every cache row against the oracle; 40 rows take the
    matrix-core prefill, 1 and 7 the row path."""
    t, p, ot, op, ox = small
    tokens, is_text = _token_rows(100 + n, n)
    kv, okv = t.new_kv(48), ot.new_kv(48)
    got = t.prefill_talker(tokens, is_text, kv)
    ref = oracle.prefill_talker(ot, ox, tokens, is_text, okv)
    print(f"prefill_talker, {n} rows ({int(is_text.sum())} text): rel err {rel_err(got, ref):.2e}")
    assert len(kv) == len(okv) == n
    assert within(got, ref)
    (gk, gv), (rk, rv) = kv.store(), okv.store()
    assert within(gk, rk) and within(gv, rv)


def test_prefill_talker_errors(ctx, small):
    t, p, ot, op, ox = small
    kv = t.new_kv(16)
    cases = (([TALKER.vocab], [False], qtts.QTTS_ERANGE), ([5, qtts.TEXT_VOCAB_1P7B], [False, True], qtts.QTTS_ERANGE),
             ([], [], qtts.QTTS_EINVAL))
    for toks, flags, status in cases:
        with pytest.raises(qtts.QttsError) as e:
            t.prefill_talker(toks, flags, kv)
        assert e.value.status == status and len(kv) == 0
    t.prefill_talker([5, 9707], [False, True], kv)
    with pytest.raises(qtts.QttsError) as e:  # the cache is no longer empty
        t.prefill_talker([5], [False], kv)
    assert e.value.status == qtts.QTTS_ESTATE and len(kv) == 2
    # a talker without text weights: codec rows only
    tw = qtts.TalkerWeights(95, TALKER)
    bare, obare = qtts.Talker(ctx, tw), oracle.Talker(tw, nthreads=1)
    kv2, okv2 = bare.new_kv(8), obare.new_kv(8)
    with pytest.raises(qtts.QttsError) as e:
        bare.prefill_talker([5, 9707], [False, True], kv2)
    assert e.value.status == qtts.QTTS_ESTATE and len(kv2) == 0
    got = bare.prefill_talker([5, 2148, 3000], [False] * 3, kv2)
    assert within(got, oracle.prefill_talker(obare, None, [5, 2148, 3000], [False] * 3, okv2))


# A decoder whose codebooks cover the talker's whole codec vocabulary, so
# every sampled semantic code decodes (the 1.7B decoder's 2048 entries do not
# cover a random-init talker's 3072).
SPEECH_DECODER = qtts.DecoderConfig(hidden=64, heads=4, head_dim=16, inter=128, window=8, codebook_dim=32,
                                    codebook_size=TALKER.vocab, vq_dim=64, latent=128, num_rest=15, layers=2,
                                    upsample=(2,), vocos_channels=96, vocos=((96, 48, 4, 2), (48, 24, 6, 3)),
                                    rope_rows=64)


@pytest.fixture(scope="module")
def speech_decoder(ctx):
    w = qtts.DecoderWeights(96, SPEECH_DECODER)
    return w, qtts.SpeechDecoder(ctx, w)


@pytest.mark.parametrize("voice", [False, True], ids=["speaker", "voice"])
def test_generate_speech_to_audio(small, speech_decoder, voice):
    """generate_speech (src/generate_new.rs:191-311) in one call: the audio is
    bit for bit the decoder's audio of generate_speech_codes's codes (same
    seed), those codes are the oracle's, and the audio is within the bar of
    the oracle's decode of them."""
    t, p, ot, op, ox = small
    w, dec = speech_decoder
    v = qtts.synth_normal_f32(97, "voice", TALKER.hidden) if voice else None
    params = qtts.loop_params(20, stop_on_eos=False)
    audio, nf = qtts.generate_speech(t, p, dec, TOKENS, SPEAKER, LANGUAGE, t.new_kv(40), p.new_kv(), params, seed=13,
                                     voice_embedding=v)
    codes = qtts.generate_speech_codes(t, p, TOKENS, SPEAKER, LANGUAGE, t.new_kv(40), p.new_kv(), params, seed=13,
                                       voice_embedding=v)
    ref_codes = ox.generate_speech_codes(op, TOKENS, SPEAKER, LANGUAGE, ot.new_kv(40), op.new_kv(), params, 13, v)
    assert nf == codes.shape[1] == 20
    assert np.array_equal(codes, ref_codes)
    assert audio.shape == (dec.num_samples(20),)
    assert np.array_equal(audio, dec.decode_to_audio(codes))
    ref = oracle.decode_to_audio(w, ref_codes)
    print(f"generate_speech, 20 frames: {audio.size} samples, rel err {rel_err(audio, ref):.2e}")
    assert within(audio, ref, tight=2e-4)


def test_generate_speech_errors(ctx, small, speech_decoder):
    t, p, ot, op, ox = small
    w, dec = speech_decoder
    params = qtts.loop_params(6, stop_on_eos=False)
    # no frames: no audio
    audio, nf = qtts.generate_speech(t, p, dec, TOKENS, SPEAKER, LANGUAGE, t.new_kv(40), p.new_kv(),
                                     qtts.loop_params(0), seed=1)
    assert nf == 0 and audio.size == 0
    # an audio buffer short of max_codes frames: refused before any work
    kv, pkv = t.new_kv(40), p.new_kv()
    out, n, nfc = np.empty(dec.num_samples(6) - 1, np.float32), C.c_int64(), C.c_int32()
    st = ctx.lib.qtts_generate_speech(t.h, p.h, dec.h, qtts._ptr(np.asarray(TOKENS, np.uint32)), len(TOKENS),
                                      SPEAKER, LANGUAGE, None, kv.h, pkv.h, C.byref(params), 1,
                                      qtts._ptr(out), out.size, C.byref(n), C.byref(nfc))
    assert st == qtts.QTTS_ERANGE and len(kv) == 0 and n.value == 0
    # a decoder whose codebook is smaller than the codes sampled: the
    # reference's lookup would panic, here QTTS_ERANGE
    small_cb = qtts.DecoderWeights(98, dataclasses.replace(SPEECH_DECODER, codebook_size=64))
    codes = qtts.generate_speech_codes(t, p, TOKENS, SPEAKER, LANGUAGE, t.new_kv(40), p.new_kv(), params, seed=3)
    assert codes.max() >= 64
    with pytest.raises(qtts.QttsError) as e:
        qtts.generate_speech(t, p, qtts.SpeechDecoder(ctx, small_cb), TOKENS, SPEAKER, LANGUAGE, t.new_kv(40),
                             p.new_kv(), params, seed=3)
    assert e.value.status == qtts.QTTS_ERANGE


@pytest.mark.timeout(600)
def test_generate_speech_codes_full(ctx):
    """The 1.7B talker, predictor and text projection (text vocab 151936,
    text hidden 2048): token ids to 8 sampled frames, codes identical."""
    tw = qtts.TalkerWeights(1, FULL_TALKER)
    pw = qtts.CodePredictorWeights(1, FULL_PREDICTOR, talker_hidden=FULL_TALKER.hidden)
    text = qtts.TextWeights(5)
    t, p = qtts.Talker(ctx, tw), qtts.CodePredictor(ctx, pw)
    t.attach_text(text)
    ot, op = oracle.Talker(tw), oracle.CodePredictor(pw)
    ox = oracle.Text(ot, text)
    params = qtts.loop_params(8, temperature=0.8, top_k=50, repetition_penalty=1.05, stop_on_eos=False)
    got = qtts.generate_speech_codes(t, p, TOKENS, SPEAKER, LANGUAGE, t.new_kv(64), p.new_kv(), params, seed=5)
    ref = ox.generate_speech_codes(op, TOKENS, SPEAKER, LANGUAGE, ot.new_kv(64), op.new_kv(), params, 5)
    assert got.shape == ref.shape == (16, 8)
    assert np.array_equal(got, ref), np.argwhere(got != ref)[:5]
