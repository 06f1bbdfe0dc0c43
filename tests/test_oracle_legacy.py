"""Pins the oracle's legacy single-step API: sample_top_k (src/generate.rs:
50-84), predict_codes (src/code_predictor.rs:126-213) and
forward_talker_decode (src/talker.rs:161-258).

sample_top_k is pinned by hand-built cases, one per rule (greedy takes the
last maximum, top-k truncation, the sorted-order inverse CDF, the k-th-entry
fallback at r == 1.0, the rng advancing only when sampling) and by the
empirical distribution of many draws against softmax(l / T) over the top k.
predict_codes is pinned against the float64 numpy model (tests/numpy_model.py)
over three appended steps, at offsets past row 4096 of its 65536-row table,
and past the end of a short table (no rotation); forward_talker_decode against the exact
composition embed_*_token -> forward_with_embedding and the float64 model."""
import dataclasses

import numpy as np
import pytest

import numpy_model as nm
import qtts
from oracle import oracle
from shapes import TINY_PREDICTOR, TINY_TALKER, rel_err

MASK = (1 << 64) - 1


def _preimage(target):
    """State s with xorshift64(s) == target (the map is a bijection)."""
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

    return unl(unr(unl(target, 17), 7), 13)


def _seed_for_r(lo, hi):
    for i in range(1, 100000):
        s = (i * 0x9E3779B97F4A7C15) & MASK
        r, _ = oracle.simple_rand(s)
        if lo <= r < hi:
            return s
    raise AssertionError("no seed found")


# ---------------------------------------------------------------- sample_top_k
@pytest.mark.parametrize("temperature", [0.0, -0.5])
def test_greedy_last_maximum_and_rng_untouched(temperature):
    logits = np.array([1.0, 3.0, 3.0, 2.0, 3.0, -1.0], dtype=np.float32)
    assert oracle.sample_top_k(logits, temperature, 50, 1234) == (4, 1234)
    assert oracle.sample_top_k(logits[:4], temperature, 0, 99) == (2, 99)  # top_k unused when greedy


def test_top1_is_the_maximum():
    logits = qtts.synth_normal_f32(3, "legacy.top1", 2048, 0.0, 3.0)
    best = int(np.argmax(logits))
    for seed in (1, 77, 0xDEADBEEF, _preimage(MASK)):
        tok, st = oracle.sample_top_k(logits, 0.9, 1, seed)
        assert tok == best
        assert st == oracle.simple_rand(seed)[1]  # one draw per sample


def test_fallback_is_the_kth_entry():
    """r == 1.0 is never below the cumulative sum: the k-th sorted entry
    (the new sampler's fallback is token 0; this one's is indices[k-1])."""
    logits = np.array([0.0, 5.0, 3.0, 4.0, 1.0], dtype=np.float32)
    seed = _preimage(MASK)
    assert oracle.simple_rand(seed)[0] == 1.0
    assert oracle.sample_top_k(logits, 1.0, 3, seed)[0] == 2
    assert oracle.sample_top_k(logits, 1.0, 4, seed)[0] == 4
    assert oracle.sample_top_k(logits, 1.0, 99, seed)[0] == 0  # k = vocab


def test_inverse_cdf_in_sorted_order():
    """p over the sorted top-k: [5 -> 0.665, 4 -> 0.245, 3 -> 0.090]; the
    draw r picks the first sorted entry whose cumulative sum exceeds r."""
    logits = np.array([0.0, 5.0, 3.0, 4.0, 1.0], dtype=np.float32)
    p = np.exp(np.array([5.0, 4.0, 3.0]) - 5.0)
    cum = np.cumsum(p / p.sum())
    order = [1, 3, 2]
    checked = 0
    for i in range(1, 400):
        seed = (i * 0x9E3779B97F4A7C15) & MASK
        r, _ = oracle.simple_rand(seed)
        if np.min(np.abs(cum - r)) < 1e-5:
            continue
        want = order[int(np.searchsorted(cum, r, side="right"))]
        assert oracle.sample_top_k(logits, 1.0, 3, seed)[0] == want, (seed, r)
        checked += 1
    assert checked > 300


def test_temperature_divides_inside_exp():
    """Top 2 of [2.0, 1.5, 1.0]: p0 = 1 / (1 + e^(-0.5 / T)) is 0.731 at
    T = 0.5 and 0.622 at T = 1 (0.562 if T multiplied).  One draw r in
    (0.64, 0.70) tells them apart."""
    logits = np.array([2.0, 1.5, 1.0], dtype=np.float32)
    seed = _seed_for_r(0.64, 0.70)
    assert oracle.sample_top_k(logits, 0.5, 2, seed)[0] == 0
    assert oracle.sample_top_k(logits, 1.0, 2, seed)[0] == 1
    assert oracle.sample_top_k(logits, 2.0, 2, seed)[0] == 1


def test_ties_by_ascending_index():
    """The reference's unstable sort leaves equal logits in an unspecified
    order; the oracle (and the device) put the lower index first."""
    logits = np.array([3.0, 3.0, 3.0, 0.0], dtype=np.float32)
    assert oracle.sample_top_k(logits, 1.0, 2, _seed_for_r(0.0, 0.49))[0] == 0
    assert oracle.sample_top_k(logits, 1.0, 2, _seed_for_r(0.51, 0.99))[0] == 1


def test_distribution_matches_truncated_softmax():
    logits = qtts.synth_normal_f32(5, "legacy.dist", 12, 0.0, 1.0)
    T, k, n = 0.7, 5, 20000
    top = np.argsort(-logits.astype(np.float64), kind="stable")[:k]
    p = np.exp((logits[top].astype(np.float64) - logits[top[0]]) / T)
    p /= p.sum()
    counts = np.zeros(logits.size)
    st = 42
    for _ in range(n):
        tok, st = oracle.sample_top_k(logits, T, k, st)
        counts[tok] += 1
    outside = np.setdiff1d(np.arange(logits.size), top)
    assert counts[outside].sum() == 0
    freq = counts[top] / n
    assert np.all(np.abs(freq - p) < 4.5 * np.sqrt(p * (1 - p) / n) + 1e-9), (freq, p)


def test_sample_top_k_failures():
    logits = np.array([0.0, np.nan, 1.0], dtype=np.float32)
    for T in (0.0, 1.0):
        with pytest.raises(oracle.OracleError) as e:
            oracle.sample_top_k(logits, T, 2, 1)
        assert e.value.status == qtts.QTTS_ENAN
    with pytest.raises(oracle.OracleError) as e:
        oracle.sample_top_k(np.zeros(4, np.float32), 1.0, 0, 1)
    assert e.value.status == qtts.QTTS_EINVAL


# ---------------------------------------------------------------- predict_codes
@pytest.fixture(scope="module")
def tiny():
    tw = qtts.TalkerWeights(41, TINY_TALKER)
    pw = qtts.CodePredictorWeights(41, TINY_PREDICTOR, talker_hidden=TINY_TALKER.hidden)
    text = qtts.TextWeights(42, qtts.TEXT_VOCAB_1P7B, 64, TINY_TALKER.hidden)
    ot = oracle.Talker(tw, nthreads=1)
    return tw, pw, text, ot, oracle.CodePredictor(pw, nthreads=1), oracle.Text(ot, text, nthreads=1)


def test_predict_codes_appends_vs_float64(tiny):
    """Three calls on one cache: offsets 0, 1, 2 (RoPE at the offset), each
    returning every head's logits of the final-normed row."""
    _, pw, _, _, op, _ = tiny
    model = nm.PredictorModel(pw)
    cache = model.stack.empty_cache()
    kv = op.new_kv(8)
    for i in range(3):
        h = qtts.synth_normal_f32(43 + i, "legacy.th", TINY_TALKER.hidden)
        got = op.predict_codes(h, kv)
        assert got.shape == (pw.num_groups, TINY_PREDICTOR.vocab) and len(kv) == i + 1
        x = model.stack.step(model.project(h), cache, i)
        normed = nm.rms_norm(x, model.final)
        ref = np.stack([normed @ hd for hd in model.heads])
        assert rel_err(got, ref) < 1e-5, i


def test_predict_codes_cache_limit(tiny):
    _, pw, _, _, op, _ = tiny
    kv = op.new_kv(2)
    h = qtts.synth_normal_f32(47, "legacy.th", TINY_TALKER.hidden)
    op.predict_codes(h, kv)
    op.predict_codes(h, kv)
    with pytest.raises(oracle.OracleError) as e:
        op.predict_codes(h, kv)
    assert e.value.status == qtts.QTTS_ERANGE and len(kv) == 2


def _history(cfg, rows, seed):
    """rows of seeded K/V history [layers][rows][kv_heads][head_dim] and the
    float64 cache of the same values."""
    k = qtts.synth_normal_f32(seed, "legacy.k", cfg.layers * rows * cfg.kv_heads * cfg.head_dim).reshape(
        cfg.layers, rows, cfg.kv_heads, cfg.head_dim)
    v = qtts.synth_normal_f32(seed, "legacy.v", k.size).reshape(k.shape)
    return k, v, [(k[i].astype(np.float64), v[i].astype(np.float64)) for i in range(cfg.layers)]


@pytest.mark.parametrize("offset", [4095, 4096, 5000])
def test_predict_codes_whole_rope_table(tiny, offset):
    """The table covers max_position rows (65536, src/loader.rs:859-874), so
    offsets past 4096 rotate too: the oracle against the float64 model, whose
    angles come from the formula directly."""
    _, pw, _, _, op, _ = tiny
    c = TINY_PREDICTOR
    assert c.max_position == 65536
    k, v, cache = _history(c, offset, 48)
    kv = op.new_kv(offset + 1)
    kv.load(k, v, offset)
    h = qtts.synth_normal_f32(49, "legacy.th", TINY_TALKER.hidden)
    got = op.predict_codes(h, kv)
    model = nm.PredictorModel(pw)
    normed = nm.rms_norm(model.stack.step(model.project(h), cache, offset), model.final)
    ref = np.stack([normed @ hd for hd in model.heads])
    assert len(kv) == offset + 1 and rel_err(got, ref) < 1e-5


def test_predict_codes_skip_past_table(monkeypatch):
    """A predictor whose table has 8 rows: offsets 8 and 9 skip the rotation
    (src/code_predictor.rs:105-107) and offset 7 still rotates; the float64
    model with its rotation switched off at those offsets."""
    c = dataclasses.replace(TINY_PREDICTOR, max_position=8)
    pw = qtts.CodePredictorWeights(51, c, talker_hidden=TINY_TALKER.hidden)
    op = oracle.CodePredictor(pw, nthreads=1)
    model = nm.PredictorModel(pw)
    rotate = nm.rope
    monkeypatch.setattr(nm, "rope", lambda x, pos, theta: x if pos >= 8 else rotate(x, pos, theta))
    k, v, _ = _history(c, 7, 52)
    kv = op.new_kv(10)
    kv.load(k, v, 7)
    cache = [(k[i].astype(np.float64), v[i].astype(np.float64)) for i in range(c.layers)]
    for offset in (7, 8, 9):
        h = qtts.synth_normal_f32(53 + offset, "legacy.th", TINY_TALKER.hidden)
        got = op.predict_codes(h, kv)
        normed = nm.rms_norm(model.stack.step(model.project(h), cache, offset), model.final)
        ref = np.stack([normed @ hd for hd in model.heads])
        assert rel_err(got, ref) < 1e-5, offset
    # and the skip is visible: rotating offset 9 instead moves the result
    monkeypatch.setattr(nm, "rope", rotate)
    cache2 = [(a[:9], b[:9]) for a, b in cache]
    h = qtts.synth_normal_f32(62, "legacy.th", TINY_TALKER.hidden)
    normed = nm.rms_norm(model.stack.step(model.project(h), cache2, 9), model.final)
    assert rel_err(got, np.stack([normed @ hd for hd in model.heads])) > 1e-3


# ---------------------------------------------------------------- forward_talker_decode
@pytest.mark.parametrize("is_text,token", [(False, 0), (False, 149), (False, TINY_TALKER.vocab - 1),
                                           (True, qtts.TTS_PAD), (True, 9707)])
def test_forward_talker_decode_composition(tiny, is_text, token):
    tw, _, text, ot, _, ox = tiny
    emb = ox.embed_text_token(token) if is_text else ot.embed_codec_token(token)
    kv, kv2 = ot.new_kv(8), ot.new_kv(8)
    for pos in range(3):
        got = ox.forward_talker_decode(token, is_text, kv, pos)
        ref = ot.forward_with_embedding(emb, kv2, pos)[: TINY_TALKER.hidden]
        assert np.array_equal(got, ref) and len(kv) == pos + 1
    # and the float64 model of the same three steps
    model = nm.TalkerModel(tw)
    cache = model.stack.empty_cache()
    for pos in range(3):
        h64 = model.forward_with_embedding(emb, cache, pos)[: TINY_TALKER.hidden]
    assert rel_err(got, h64) < 1e-5


def test_forward_talker_decode_ranges(tiny):
    _, _, _, ot, _, ox = tiny
    kv = ot.new_kv(4)
    for tok, is_text in ((TINY_TALKER.vocab, False), (qtts.TEXT_VOCAB_1P7B, True)):
        with pytest.raises(oracle.OracleError) as e:
            ox.forward_talker_decode(tok, is_text, kv, 0)
        assert e.value.status == qtts.QTTS_ERANGE and len(kv) == 0
