"""GPU parity of the legacy single-step API against the oracle:
sample_top_k (src/generate.rs:50-84) on the device, predict_codes
(src/code_predictor.rs:126-213) appending to a persistent predictor cache,
and forward_talker_decode (src/talker.rs:161-258) fed codec and text tokens,
on small models and at the 1.7B shapes; predict_codes past row 4096 of the
65536-row RoPE table and past the end of an 8-row one.

Bars: tokens and rng states identical (tie-free logits: the reference leaves
the order of equal logits unspecified); hidden states, logits and cache rows
within 1e-3 relative (the GEMVs sum in another order than the oracle's)."""
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
TOL = 1e-3
MASK = (1 << 64) - 1


def _preimage_of_mask():
    """The xorshift64 state whose next state is 2^64 - 1 (simple_rand gives 1.0)."""
    def unl(y, k):
        x = y
        for _ in range(64 // k + 1):
            x = y ^ ((x << k) & MASK)
        return x

    def unr(y, k):
        x = y
        for _ in range(64 // k + 1):
            x = y ^ (x >> k)
        return x

    return unl(unr(unl(MASK, 17), 7), 13)


# ---------------------------------------------------------------- sample_top_k
@pytest.mark.parametrize("vocab", [1, 7, 256, 2048, 3072, 4096])
def test_sample_top_k_matches_oracle(ctx, vocab):
    logits = qtts.synth_normal_f32(vocab, "legacy.topk", vocab, 0.0, 2.5)
    assert np.unique(logits).size == vocab  # tie-free
    cases = [(0.0, 50), (-1.0, 0), (0.7, 1), (0.7, 50), (1.3, 5), (0.9, vocab), (0.9, vocab + 9), (0.05, 3)]
    for T, k in cases:
        for seed in (1, 0x1234567, 0xDEADBEEFCAFE, (vocab * 0x9E3779B97F4A7C15) & MASK, _preimage_of_mask()):
            got = ctx.sample_top_k(logits, T, k, seed)
            ref = oracle.sample_top_k(logits, T, k, seed)
            assert got == ref, (T, k, seed)


def test_sample_top_k_sequence(ctx):
    """1000 chained draws (the rng carried from call to call)."""
    logits = qtts.synth_normal_f32(3, "legacy.seq", 2048, 0.0, 1.5)
    g = r = 77
    for i in range(1000):
        tg, g = ctx.sample_top_k(logits, 0.8, 50, g)
        tr, r = oracle.sample_top_k(logits, 0.8, 50, r)
        assert (tg, g) == (tr, r), i


def test_sample_top_k_failures(ctx):
    bad = np.array([0.0, np.nan, 1.0], dtype=np.float32)
    for T in (0.0, 1.0):
        with pytest.raises(qtts.QttsError) as e:
            ctx.sample_top_k(bad, T, 2, 1)
        assert e.value.status == qtts.QTTS_ENAN
    with pytest.raises(qtts.QttsError) as e:
        ctx.sample_top_k(np.zeros(4, np.float32), 1.0, 0, 1)
    assert e.value.status == qtts.QTTS_EINVAL
    with pytest.raises(qtts.QttsError) as e:
        ctx.sample_top_k(np.zeros(4097, np.float32), 1.0, 5, 1)
    assert e.value.status == qtts.QTTS_ESHAPE
    # the context still works afterwards
    assert ctx.sample_top_k(np.arange(5, dtype=np.float32), 0.0, 1, 3) == (4, 3)


# ---------------------------------------------------------------- predict_codes
@pytest.fixture(scope="module")
def small(ctx):
    tw = qtts.TalkerWeights(61, TALKER)
    pw = qtts.CodePredictorWeights(61, PREDICTOR, talker_hidden=TALKER.hidden)
    text = qtts.TextWeights(62, qtts.TEXT_VOCAB_1P7B, 64, TALKER.hidden)
    t, p = qtts.Talker(ctx, tw), qtts.CodePredictor(ctx, pw)
    t.attach_text(text)
    ot, op = oracle.Talker(tw, nthreads=1), oracle.CodePredictor(pw, nthreads=1)
    return t, p, ot, op, oracle.Text(ot, text, nthreads=1)


def _predict_steps(p, op, steps, seed, talker_hidden, cap=32):
    kv, okv = p.new_kv(cap), op.new_kv(cap)
    for i in range(steps):
        h = qtts.synth_normal_f32(seed + i, "legacy.th", talker_hidden)
        got, ref = p.predict_codes(h, kv), op.predict_codes(h, okv)
        assert got.shape == ref.shape
        assert within(got, ref), i
        assert len(kv) == len(okv) == i + 1
    (gk, gv), (rk, rv) = kv.store(), okv.store()
    assert within(gk, rk) and within(gv, rv)


def test_predict_codes_small(small):
    t, p, ot, op, ox = small
    _predict_steps(p, op, 20, 63, TALKER.hidden)


def test_predict_codes_limits(small):
    t, p, ot, op, ox = small
    h = qtts.synth_normal_f32(64, "legacy.th", TALKER.hidden)
    kv = p.new_kv(2)
    p.predict_codes(h, kv)
    p.predict_codes(h, kv)
    with pytest.raises(qtts.QttsError) as e:
        p.predict_codes(h, kv)
    assert e.value.status == qtts.QTTS_ERANGE and len(kv) == 2


@pytest.mark.parametrize("offset", [4095, 4096, 5000])
def test_predict_codes_whole_rope_table(small, offset):
    """The device table holds all max_position = 65536 rows
    (src/loader.rs:859-874): offsets past 4096 rotate like the oracle's."""
    t, p, ot, op, ox = small
    c = PREDICTOR
    h = qtts.synth_normal_f32(64, "legacy.th", TALKER.hidden)
    kv, okv = p.new_kv(offset + 1), op.new_kv(offset + 1)
    z = qtts.synth_normal_f32(65, "legacy.kv", c.layers * offset * c.kv_heads * c.head_dim).reshape(
        c.layers, offset, c.kv_heads, c.head_dim)
    kv.load(z, z, offset)
    okv.load(z, z, offset)
    got, ref = p.predict_codes(h, kv), op.predict_codes(h, okv)
    print(f"predict_codes at offset {offset}: rel err {rel_err(got, ref):.2e}")
    assert within(got, ref) and len(kv) == offset + 1
    (gk, gv), (rk, rv) = kv.store(), okv.store()
    assert within(gk[:, offset], rk[:, offset]) and within(gv[:, offset], rv[:, offset])


def test_predict_codes_skip_past_table(ctx):
    """A predictor with an 8-row table: offsets 8 and 9 skip the rotation
    (src/code_predictor.rs:105-107), offset 7 rotates; as the oracle does."""
    c = dataclasses.replace(PREDICTOR, max_position=8)
    pw = qtts.CodePredictorWeights(66, c, talker_hidden=TALKER.hidden)
    p, op = qtts.CodePredictor(ctx, pw), oracle.CodePredictor(pw, nthreads=1)
    z = qtts.synth_normal_f32(67, "legacy.kv", c.layers * 7 * c.kv_heads * c.head_dim).reshape(
        c.layers, 7, c.kv_heads, c.head_dim)
    kv, okv = p.new_kv(10), op.new_kv(10)
    kv.load(z, z, 7)
    okv.load(z, z, 7)
    for offset in (7, 8, 9):
        h = qtts.synth_normal_f32(68 + offset, "legacy.th", TALKER.hidden)
        assert within(p.predict_codes(h, kv), op.predict_codes(h, okv)), offset
    (gk, gv), (rk, rv) = kv.store(), okv.store()
    assert within(gk, rk) and within(gv, rv)


@pytest.mark.timeout(600)
def test_predict_codes_full(ctx):
    """The 1.7B predictor (5 layers, hidden 1024, 15 heads of 2048)."""
    pw = qtts.CodePredictorWeights(7, FULL_PREDICTOR, talker_hidden=FULL_TALKER.hidden)
    p, op = qtts.CodePredictor(ctx, pw), oracle.CodePredictor(pw)
    _predict_steps(p, op, 4, 66, FULL_TALKER.hidden, cap=16)


# ---------------------------------------------------------------- forward_talker_decode
@pytest.mark.parametrize("is_text,token", [(False, 0), (False, qtts.CODEC_BOS), (False, TALKER.vocab - 1),
                                           (True, qtts.TTS_PAD), (True, 9707), (True, qtts.TEXT_VOCAB_1P7B - 1)])
def test_forward_talker_decode_small(small, is_text, token):
    t, p, ot, op, ox = small
    kv, okv, kv2 = t.new_kv(16), ot.new_kv(16), t.new_kv(16)
    emb = t.embed_text_token(token) if is_text else t.embed_codec_token(token)
    for pos in range(4):
        got = t.forward_talker_decode(token, is_text, kv, pos)
        ref = ox.forward_talker_decode(token, is_text, okv, pos)
        assert within(got, ref), pos
        # the same step through forward_with_embedding on the device
        both = t.forward_with_embedding(emb, kv2, pos)
        assert np.array_equal(got, both[: TALKER.hidden]), pos
    (gk, gv), (rk, rv) = kv.store(), okv.store()
    assert within(gk, rk) and within(gv, rv)


def test_forward_talker_decode_errors(small, ctx):
    t, p, ot, op, ox = small
    kv = t.new_kv(4)
    for tok, is_text in ((TALKER.vocab, False), (qtts.TEXT_VOCAB_1P7B, True)):
        with pytest.raises(qtts.QttsError) as e:
            t.forward_talker_decode(tok, is_text, kv, 0)
        assert e.value.status == qtts.QTTS_ERANGE and len(kv) == 0
    bare = qtts.Talker(ctx, qtts.TalkerWeights(67, TALKER))  # no text weights
    with pytest.raises(qtts.QttsError) as e:
        bare.forward_talker_decode(qtts.TTS_PAD, True, bare.new_kv(4), 0)
    assert e.value.status == qtts.QTTS_ESTATE
    bare.close()


@pytest.mark.timeout(600)
def test_forward_talker_decode_full(ctx):
    """The 1.7B talker with the 1.7B text projection: a text step then two
    codec steps."""
    tw = qtts.TalkerWeights(8, FULL_TALKER)
    text = qtts.TextWeights(9)
    t = qtts.Talker(ctx, tw)
    t.attach_text(text)
    ot = oracle.Talker(tw)
    ox = oracle.Text(ot, text)
    kv, okv = t.new_kv(8), ot.new_kv(8)
    for pos, (tok, is_text) in enumerate(((qtts.TTS_BOS, True), (qtts.CODEC_BOS, False), (1234, False))):
        got = t.forward_talker_decode(tok, is_text, kv, pos)
        ref = ox.forward_talker_decode(tok, is_text, okv, pos)
        assert within(got, ref), pos
