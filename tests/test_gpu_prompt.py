"""GPU parity of the prompt assembly on the device against the oracle:
embed_text_token (src/talker.rs:105-116), the rows of prefill_custom_voice
(src/generate_new.rs:60-177, built-in speaker and voice-embedding paths),
the prefill itself (src/generate_new.rs:84-188), build_trailing_text
(src/generate_new.rs:314-326), and generate_speech from token ids to codes
(src/generate_new.rs:191-300) with no embedding math on the host: a small
model with the real codec and text vocabularies, and the 1.7B talker and
predictor with the 1.7B text projection.

Bars: rows, hidden states and logits within 1e-3 relative (the text
projection's GEMV sums in another order than the oracle's); codes identical."""
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
