"""GPU parity of the composite paths — talker decode step, talker prefill,
predictor frame and the frame loop — against the oracle on the same seeded
random-init weights and inputs.

Bars: hidden states and logits within REL_TOL = 1e-3 relative (fp32
accumulate) and within the regression bar of tests/shapes.py (about ten
times the measured error); predictor codes and greedy loop codes identical.
"""
import time

import numpy as np
import pytest

import qtts
from oracle import oracle
from shapes import FULL_PREDICTOR, FULL_TALKER, TINY_PREDICTOR, TINY_TALKER, rel_err, within

pytestmark = pytest.mark.gpu

REL_TOL = 1e-3


@pytest.fixture(scope="module")
def tiny(ctx):
    tw = qtts.TalkerWeights(21, TINY_TALKER)
    pw = qtts.CodePredictorWeights(21, TINY_PREDICTOR, talker_hidden=TINY_TALKER.hidden)
    return tw, pw, qtts.Talker(ctx, tw), qtts.CodePredictor(ctx, pw), oracle.Talker(tw, 1), oracle.CodePredictor(pw, 1)


@pytest.fixture(scope="module")
def full(ctx):
    t0 = time.time()
    tw = qtts.TalkerWeights(1, FULL_TALKER)
    pw = qtts.CodePredictorWeights(1, FULL_PREDICTOR, talker_hidden=FULL_TALKER.hidden)
    print(f"synthetic 1.7B weights in {time.time() - t0:.1f}s", flush=True)
    return tw, pw, qtts.Talker(ctx, tw), qtts.CodePredictor(ctx, pw), oracle.Talker(tw), oracle.CodePredictor(pw)


def test_talker_steps_tiny(tiny):
    tw, _, t, _, ot, _ = tiny
    cfg = tw.cfg
    kv, okv = t.new_kv(40), ot.new_kv(40)
    for step in range(20):
        emb = qtts.synth_normal_f32(22, f"tiny.emb.{step}", cfg.hidden)
        got = t.forward_with_embedding(emb, kv, step + 3)
        ref = ot.forward_with_embedding(emb, okv, step + 3)
        assert within(got[: cfg.hidden], ref[: cfg.hidden])
        assert within(got[cfg.hidden:], ref[cfg.hidden:])
    assert len(kv) == len(okv) == 20
    k, v = kv.store()
    ok, ov = okv.store()
    assert within(k, ok) and within(v, ov)


def test_talker_step_full_prefilled_kv(full):
    """Single talker decode step: 28 layers, KV pre-filled to 256 positions
    with N(0,1), one N(0,1) embedding at position 256."""
    tw, _, t, _, ot, _ = full
    cfg = tw.cfg
    L = 256
    shape = (cfg.layers, L, cfg.kv_heads, cfg.head_dim)
    k = qtts.synth_normal_f32(3, "kv.k", int(np.prod(shape))).reshape(shape)
    v = qtts.synth_normal_f32(3, "kv.v", int(np.prod(shape))).reshape(shape)
    kv, okv = t.new_kv(1024), ot.new_kv(1024)
    kv.load(k, v, L)
    okv.load(k, v, L)
    emb = qtts.synth_normal_f32(3, "step.emb", cfg.hidden)
    got = t.forward_with_embedding(emb, kv, L)
    ref = ot.forward_with_embedding(emb, okv, L)
    eh, el = rel_err(got[: cfg.hidden], ref[: cfg.hidden]), rel_err(got[cfg.hidden:], ref[cfg.hidden:])
    print(f"full talker step: hidden rel err {eh:.2e}, logits rel err {el:.2e}")
    assert within(got[: cfg.hidden], ref[: cfg.hidden]) and within(got[cfg.hidden:], ref[cfg.hidden:])
    assert int(np.argmax(got[cfg.hidden:])) == int(np.argmax(ref[cfg.hidden:]))


@pytest.mark.parametrize("seq_len", [1, 5, 13, 70, 300, 700])
def test_prefill_tiny(tiny, seq_len):
    """Below 8 rows the prefill runs on the GEMV path, from 8 rows on the
    matrix cores (70 rows: two 64-row GEMM passes).  Past 256 rows the causal
    attention splits each row's positions into 256-position pieces merged by
    the last split (300 rows: 2 splits; 700 rows: 3, and the rows in two
    attention launches of at most 512)."""
    tw, _, t, _, ot, _ = tiny
    cfg = tw.cfg
    x = qtts.synth_normal_f32(23, f"prefill.{seq_len}", seq_len * cfg.hidden)
    cap = max(32, seq_len + 8)
    kv, okv = t.new_kv(cap), ot.new_kv(cap)
    got = t.prefill_talker_raw(x, seq_len, kv)
    ref = ot.prefill_talker_raw(x, seq_len, okv)
    assert within(got, ref)
    k, v = kv.store()
    ok, ov = okv.store()
    assert within(k, ok) and within(v, ov)
    # a decode step continues from the prefilled cache
    emb = qtts.synth_normal_f32(23, "prefill.next", cfg.hidden)
    assert within(t.forward_with_embedding(emb, kv, seq_len), ot.forward_with_embedding(emb, okv, seq_len))


def test_prefill_nonempty_cache_rejected(tiny):
    tw, _, t, _, _, _ = tiny
    kv = t.new_kv(8)
    t.forward_with_embedding(np.zeros(tw.cfg.hidden, np.float32), kv, 0)
    with pytest.raises(qtts.QttsError) as e:
        t.prefill_talker_raw(np.zeros(2 * tw.cfg.hidden, np.float32), 2, kv)
    assert e.value.status == qtts.QTTS_ESTATE


def test_prefill_full_64(full):
    tw, _, t, _, ot, _ = full
    x = qtts.synth_normal_f32(4, "prefill64", 64 * tw.cfg.hidden)
    kv, okv = t.new_kv(128), ot.new_kv(128)
    got = t.prefill_talker_raw(x, 64, kv)
    ref = ot.prefill_talker_raw(x, 64, okv)
    print(f"prefill 64 rel err {rel_err(got, ref):.2e}")
    assert within(got, ref)


def test_predictor_tiny(tiny):
    tw, pw, t, p, ot, op = tiny
    for i in range(6):
        h = qtts.synth_normal_f32(24, f"ph.{i}", tw.cfg.hidden)
        sem = ot.embed_codec_token(100 + i)
        got = p.generate_acoustic_codes(h, sem, p.new_kv())
        ref = op.generate_acoustic_codes(h, sem, op.new_kv())
        assert np.array_equal(got, ref), (got, ref)
        assert np.array_equal(p.get_acoustic_embeddings_sum(got), op.get_acoustic_embeddings_sum(ref))


@pytest.mark.parametrize("capacity", [16, 40])
def test_predictor_cache_paths(tiny, capacity):
    """Both predictor paths: the frame engine with the cached rows kept in
    the LDS of the blocks that run the layer (capacity <= 32), and, for a
    larger capacity (the first pass's two rows then exceed the engine's
    attention outside LDS), the multi-kernel path reading the rows back from
    the device cache.  Codes match, and so does the cache the call leaves for
    the host."""
    tw, pw, t, p, ot, op = tiny
    for i in range(3):
        h = qtts.synth_normal_f32(31, f"pc.{i}", tw.cfg.hidden)
        sem = ot.embed_codec_token(50 + i)
        kv, okv = p.new_kv(capacity), op.new_kv(capacity)
        got = p.generate_acoustic_codes(h, sem, kv)
        ref = op.generate_acoustic_codes(h, sem, okv)
        assert np.array_equal(got, ref), (got, ref)
        (gk, gv), (rk, rv) = kv.store(), okv.store()
        assert gk.shape == rk.shape
        assert within(gk, rk) and within(gv, rv)


def test_predictor_full(full):
    tw, pw, t, p, ot, op = full
    for i in range(3):
        h = qtts.synth_normal_f32(5, f"fph.{i}", tw.cfg.hidden)
        sem = ot.embed_codec_token(7 + 300 * i)
        got = p.generate_acoustic_codes(h, sem, p.new_kv())
        ref = op.generate_acoustic_codes(h, sem, op.new_kv())
        assert np.array_equal(got, ref), (got, ref)


def test_predictor_input_table_on_and_off(ctx, full, monkeypatch):
    """Passes 2-15 read their input row from the per-code table of projected
    embeddings (the default); QTTS_PREDICTOR_TABLE=0, read when a predictor
    first runs, keeps the projection as a step of its own.  Both give the
    oracle's codes, and their caches agree."""
    tw, pw, t, p, ot, op = full
    monkeypatch.setenv("QTTS_PREDICTOR_TABLE", "0")
    p_off = qtts.CodePredictor(ctx, pw)
    for i in range(2):
        h = qtts.synth_normal_f32(8, f"tab.{i}", tw.cfg.hidden)
        sem = ot.embed_codec_token(11 + 500 * i)
        kv_on, kv_off = p.new_kv(), p_off.new_kv()
        on = p.generate_acoustic_codes(h, sem, kv_on)
        off = p_off.generate_acoustic_codes(h, sem, kv_off)
        ref = op.generate_acoustic_codes(h, sem, op.new_kv())
        assert np.array_equal(on, ref) and np.array_equal(off, ref), (on, off, ref)
        (k1, v1), (k0, v0) = kv_on.store(), kv_off.store()
        assert within(k1, k0) and within(v1, v0)


def _loop_inputs(tw, seed, trailing=3):
    hidden = tw.cfg.hidden
    last_hidden = qtts.synth_normal_f32(seed, "loop.h", hidden)
    trailing_text = qtts.synth_normal_f32(seed, "loop.text", trailing * hidden, 0.0, 0.1).reshape(trailing, hidden)
    pad = qtts.synth_normal_f32(seed, "loop.pad", hidden, 0.0, 0.1)
    return last_hidden, trailing_text, pad


@pytest.mark.parametrize("greedy", [True, False])
def test_loop_tiny(tiny, greedy):
    tw, pw, t, p, ot, op = tiny
    last_hidden, text, pad = _loop_inputs(tw, 25)
    frames = 64
    params = qtts.loop_params(frames, greedy=greedy, stop_on_eos=False)
    kv, okv = t.new_kv(96), ot.new_kv(96)
    # start from a short prefill, as generate_speech does
    x = qtts.synth_normal_f32(25, "loop.prefill", 10 * tw.cfg.hidden)
    lh = t.prefill_talker_raw(x, 10, kv)
    olh = ot.prefill_talker_raw(x, 10, okv)
    logits = ot.apply_codec_head(olh)
    got = qtts.generate_codes(t, p, kv, p.new_kv(), olh, logits, 10, text, pad, params, seed=777)
    ref = oracle.generate_codes(ot, op, okv, op.new_kv(), olh, logits, 10, text, pad, params, seed=777)
    assert got.shape == ref.shape == (16, frames)
    assert np.array_equal(got, ref), np.argwhere(got != ref)[:5]
    assert len(kv) == len(okv) == 10 + frames
    assert within(lh, olh)


def test_engine_swiglu_full_panels(ctx, tiny, monkeypatch):
    """QTTS_ENGINE_SWIGLU_COLS=32 (read when a frame program is built) runs
    the predictor's SwiGLU step in whole-panel tasks instead of half panels:
    a predictor made with it gives the oracle's codes over a sampled loop."""
    tw, pw, _, _, ot, op = tiny
    monkeypatch.setenv("QTTS_ENGINE_SWIGLU_COLS", "32")
    t, p = qtts.Talker(ctx, tw), qtts.CodePredictor(ctx, pw)
    last_hidden, text, pad = _loop_inputs(tw, 33)
    logits = ot.apply_codec_head(last_hidden)
    params = qtts.loop_params(24, temperature=0.8, top_k=50, repetition_penalty=1.05, stop_on_eos=False)
    kv, okv = t.new_kv(32), ot.new_kv(32)
    got = qtts.generate_codes(t, p, kv, p.new_kv(), last_hidden, logits, 0, text, pad, params, seed=53)
    ref = oracle.generate_codes(ot, op, okv, op.new_kv(), last_hidden, logits, 0, text, pad, params, seed=53)
    assert np.array_equal(got, ref), np.argwhere(got != ref)[:5]
    kv.close()


def test_engine_tag_restart(tiny, monkeypatch):
    """The frame engine's 32-bit hand-off tags (8192 per code) run out every
    524,288 codes of a context; it then restarts them in a new epoch after
    clearing every tagged word.  A context whose tags start 40 codes before
    the end runs a 64-frame loop across the restart (launches of 16 codes),
    a talker step, and a second loop in the new epoch: codes, cache rows and
    step outputs match the oracle's."""
    tw, pw, _, _, ot, op = tiny
    monkeypatch.setenv("QTTS_ENGINE_TAG_START", str(0xFFFFFFFF - 40 * 8192))
    monkeypatch.delenv("QTTS_ENGINE_CODES", raising=False)
    monkeypatch.delenv("QTTS_ENGINE", raising=False)
    c = qtts.Context(0)
    try:
        t, p = qtts.Talker(c, tw), qtts.CodePredictor(c, pw)
        last_hidden, text, pad = _loop_inputs(tw, 29)
        logits = ot.apply_codec_head(last_hidden)
        params = qtts.loop_params(64, temperature=0.8, top_k=50, repetition_penalty=1.05, stop_on_eos=False)
        kv, okv = t.new_kv(96), ot.new_kv(96)
        got = qtts.generate_codes(t, p, kv, p.new_kv(), last_hidden, logits, 0, text, pad, params, seed=41)
        ref = oracle.generate_codes(ot, op, okv, op.new_kv(), last_hidden, logits, 0, text, pad, params, seed=41)
        assert got.shape == ref.shape == (16, 64)
        assert np.array_equal(got, ref), np.argwhere(got != ref)[:5]
        (k, v), (ok, ov) = kv.store(), okv.store()
        assert within(k, ok) and within(v, ov)
        emb = qtts.synth_normal_f32(29, "restart.emb", tw.cfg.hidden)
        assert within(t.forward_with_embedding(emb, kv, 64), ot.forward_with_embedding(emb, okv, 64))
        params = qtts.loop_params(24, temperature=0.8, top_k=50, repetition_penalty=1.05, stop_on_eos=False)
        kv2, okv2 = t.new_kv(32), ot.new_kv(32)
        got = qtts.generate_codes(t, p, kv2, p.new_kv(), last_hidden, logits, 0, text, pad, params, seed=43)
        ref = oracle.generate_codes(ot, op, okv2, op.new_kv(), last_hidden, logits, 0, text, pad, params, seed=43)
        assert np.array_equal(got, ref), np.argwhere(got != ref)[:5]
        for x in (kv, kv2):
            x.close()
    finally:
        c.close()


@pytest.mark.parametrize("per_launch", ["1", "7", None])
def test_loop_tiny_codes_per_launch(tiny, monkeypatch, per_launch):
    """The frame engine runs up to 16 codes per cooperative launch with a grid
    barrier between codes (QTTS_ENGINE_CODES overrides the count): 1, 7 and
    the default give the oracle's codes, cache length and cache rows, and an
    EOS that falls inside a launch stops the loop at the same frame."""
    tw, pw, t, p, ot, op = tiny
    if per_launch is None:
        monkeypatch.delenv("QTTS_ENGINE_CODES", raising=False)
    else:
        monkeypatch.setenv("QTTS_ENGINE_CODES", per_launch)
    last_hidden, text, pad = _loop_inputs(tw, 27)
    logits = ot.apply_codec_head(last_hidden)
    frames = 40
    params = qtts.loop_params(frames, temperature=0.8, top_k=50, repetition_penalty=1.05, stop_on_eos=False)
    kv, okv = t.new_kv(48), ot.new_kv(48)
    got = qtts.generate_codes(t, p, kv, p.new_kv(), last_hidden, logits, 0, text, pad, params, seed=31)
    ref = oracle.generate_codes(ot, op, okv, op.new_kv(), last_hidden, logits, 0, text, pad, params, seed=31)
    assert got.shape == ref.shape == (16, frames)
    assert np.array_equal(got, ref), np.argwhere(got != ref)[:5]
    assert len(kv) == len(okv) == frames
    (k, v), (ok, ov) = kv.store(), okv.store()
    assert k.shape == ok.shape and within(k, ok) and within(v, ov)
    # EOS at frame 20's code 0: inside the second launch of 16, the third of 7
    eos = int(ref[0, 20])
    first = int(np.argmax(ref[0] == eos))
    params = qtts.loop_params(frames, temperature=0.8, top_k=50, repetition_penalty=1.05, stop_on_eos=True,
                              codec_eos_id=eos)
    kv = t.new_kv(48)
    got = qtts.generate_codes(t, p, kv, p.new_kv(), last_hidden, logits, 0, text, pad, params, seed=31)
    assert got.shape == (16, first)
    assert np.array_equal(got, ref[:, :first])
    assert len(kv) == first


def test_loop_tiny_talker_only_and_eos(tiny):
    tw, _, t, _, ot, _ = tiny
    hidden = tw.cfg.hidden
    lh = qtts.synth_normal_f32(26, "eos.h", hidden)
    logits = ot.apply_codec_head(lh)
    params = qtts.loop_params(24, greedy=True, stop_on_eos=False, talker_only=True)
    kv, okv = t.new_kv(32), ot.new_kv(32)
    got = qtts.generate_codes(t, None, kv, None, lh, logits, 0, None, None, params, seed=1)
    ref = oracle.generate_codes(ot, None, okv, None, lh, logits, 0, None, None, params, seed=1)
    assert np.array_equal(got, ref)
    # declare the 6th frame's code EOS: both stop before that frame
    eos = int(ref[0, 5])
    first = int(np.argmax(ref[0] == eos))
    params = qtts.loop_params(24, greedy=True, stop_on_eos=True, talker_only=True, codec_eos_id=eos)
    kv, okv = t.new_kv(32), ot.new_kv(32)
    got = qtts.generate_codes(t, None, kv, None, lh, logits, 0, None, None, params, seed=1)
    ref2 = oracle.generate_codes(ot, None, okv, None, lh, logits, 0, None, None, params, seed=1)
    assert got.shape[1] == ref2.shape[1] == first
    assert np.array_equal(got, ref2)
    assert len(kv) == len(okv) == first


def test_loop_full_greedy(full):
    """Full 1.7B talker + predictor, greedy, 16 frames against the oracle."""
    tw, pw, t, p, ot, op = full
    last_hidden, text, pad = _loop_inputs(tw, 27)
    logits = ot.apply_codec_head(last_hidden)
    frames = 16
    params = qtts.loop_params(frames, greedy=True, stop_on_eos=False)
    kv, okv = t.new_kv(256), ot.new_kv(256)
    got = qtts.generate_codes(t, p, kv, p.new_kv(), last_hidden, logits, 0, text, pad, params, seed=9)
    ref = oracle.generate_codes(ot, op, okv, op.new_kv(), last_hidden, logits, 0, text, pad, params, seed=9)
    assert np.array_equal(got, ref), np.argwhere(got != ref)[:5]
