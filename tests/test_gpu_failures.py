"""The loops' failure paths on the GPU, where the reference panics
(src/code_predictor.rs:331 sample_argmax's partial_cmp().unwrap(),
src/generate_new.rs:365 sample_token's sort) or grows past its tables:

- NaN logits reaching the code-0 sampler, and a NaN hidden state reaching
  the predictor's argmax, come back as QTTS_ENAN from the frame engine, from
  the multi-kernel path (QTTS_ENGINE=ops) and from the batched loop.  Every
  kernel leaves through its abort word and exits normally; the caches keep
  their length and a clean loop on the same context afterwards gives the
  oracle's codes.
- Positions past the RoPE table and caches too small for max_codes come back
  as QTTS_ERANGE before anything is launched.
"""
import numpy as np
import pytest

import qtts
from oracle import oracle
from shapes import TINY_PREDICTOR, TINY_TALKER

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def tiny(ctx):
    tw = qtts.TalkerWeights(71, TINY_TALKER)
    pw = qtts.CodePredictorWeights(71, TINY_PREDICTOR, talker_hidden=TINY_TALKER.hidden)
    return (tw, pw, qtts.Talker(ctx, tw), qtts.CodePredictor(ctx, pw), oracle.Talker(tw, nthreads=1),
            oracle.CodePredictor(pw, nthreads=1))


def _inputs(tw, ot, seed):
    H = tw.cfg.hidden
    lh = qtts.synth_normal_f32(seed, "fail.h", H)
    text = qtts.synth_normal_f32(seed, "fail.text", 2 * H, 0.0, 0.1).reshape(2, H)
    pad = qtts.synth_normal_f32(seed, "fail.pad", H, 0.0, 0.1)
    return lh, ot.apply_codec_head(lh), text, pad


def _clean_loop_matches(tiny, seed):
    tw, pw, t, p, ot, op = tiny
    lh, lg, text, pad = _inputs(tw, ot, seed)
    params = qtts.loop_params(8, stop_on_eos=False)
    kv, okv = t.new_kv(16), ot.new_kv(16)
    got = qtts.generate_codes(t, p, kv, p.new_kv(), lh, lg, 0, text, pad, params, seed=3)
    ref = oracle.generate_codes(ot, op, okv, op.new_kv(), lh, lg, 0, text, pad, params, seed=3)
    assert np.array_equal(got, ref)


@pytest.mark.parametrize("engine", ["frame", "ops"])
@pytest.mark.parametrize("where", ["logits", "hidden"])
def test_loop_nan_is_enan(tiny, monkeypatch, engine, where):
    tw, pw, t, p, ot, op = tiny
    if engine == "ops":
        monkeypatch.setenv("QTTS_ENGINE", "ops")
    lh, lg, text, pad = _inputs(tw, ot, 72)
    if where == "logits":
        lg = lg.copy()
        lg[17] = np.nan  # the sampler's softmax turns every score NaN
    else:
        lh = lh.copy()
        lh[5] = np.nan  # the predictor's input: every logit of its first head is NaN
    # the oracle fails the same way
    okv = ot.new_kv(16)
    with pytest.raises(oracle.OracleError) as oe:
        oracle.generate_codes(ot, op, okv, op.new_kv(), lh, lg, 0, text, pad, qtts.loop_params(6), seed=1)
    assert oe.value.status == qtts.QTTS_ENAN
    kv = t.new_kv(16)
    with pytest.raises(qtts.QttsError) as e:
        qtts.generate_codes(t, p, kv, p.new_kv(), lh, lg, 0, text, pad, qtts.loop_params(6, stop_on_eos=False),
                            seed=1)
    assert e.value.status == qtts.QTTS_ENAN
    assert len(kv) == 0
    monkeypatch.delenv("QTTS_ENGINE", raising=False)
    _clean_loop_matches(tiny, 73)


def test_talker_only_nan_is_enan(tiny):
    tw, _, t, _, ot, _ = tiny
    lh, lg, _, _ = _inputs(tw, ot, 74)
    lg = lg.copy()
    lg[:] = np.nan
    kv = t.new_kv(16)
    params = qtts.loop_params(6, greedy=True, stop_on_eos=False, talker_only=True)
    with pytest.raises(qtts.QttsError) as e:
        qtts.generate_codes(t, None, kv, None, lh, lg, 0, None, None, params, seed=1)
    assert e.value.status == qtts.QTTS_ENAN
    assert len(kv) == 0
    _clean_loop_matches(tiny, 75)


def test_batch_nan_is_enan(tiny):
    """One stream of three gets NaN logits: the batched call returns
    QTTS_ENAN, no cache length moves, and a clean batch runs afterwards."""
    tw, pw, t, p, ot, op = tiny
    H = tw.cfg.hidden
    B = 3
    lh = qtts.synth_normal_f32(76, "bnan.h", B * H).reshape(B, H)
    lg = np.stack([ot.apply_codec_head(lh[b]) for b in range(B)])
    text = qtts.synth_normal_f32(76, "bnan.text", B * 2 * H, 0.0, 0.1).reshape(B, 2, H)
    pad = qtts.synth_normal_f32(76, "bnan.pad", H, 0.0, 0.1)
    params = qtts.loop_params(5, stop_on_eos=False)
    bad = lg.copy()
    bad[1, 3] = np.nan
    kvs = [t.new_kv(16) for _ in range(B)]
    with pytest.raises(qtts.QttsError) as e:
        qtts.generate_codes_batch(t, p, kvs, lh, bad, [0] * B, text, pad, params, [1, 2, 3])
    assert e.value.status == qtts.QTTS_ENAN
    assert [len(kv) for kv in kvs] == [0] * B
    kvs = [t.new_kv(16) for _ in range(B)]
    got = qtts.generate_codes_batch(t, p, kvs, lh, lg, [0] * B, text, pad, params, [1, 2, 3])
    for b in range(B):
        ref = oracle.generate_codes(ot, op, ot.new_kv(16), op.new_kv(), lh[b], lg[b], 0, text[b], pad, params,
                                    seed=1 + b)
        assert np.array_equal(got[b], ref), b


def test_erange_positions_and_capacity(tiny):
    tw, pw, t, p, ot, op = tiny
    lh, lg, text, pad = _inputs(tw, ot, 77)
    max_pos = tw.cfg.max_position
    params = qtts.loop_params(10, stop_on_eos=False)
    # positions past the RoPE table
    kv = t.new_kv(16)
    with pytest.raises(qtts.QttsError) as e:
        qtts.generate_codes(t, p, kv, p.new_kv(), lh, lg, max_pos - 5, text, pad, params, seed=1)
    assert e.value.status == qtts.QTTS_ERANGE
    with pytest.raises(qtts.QttsError) as e:
        qtts.generate_codes_batch(t, p, [kv], lh[None], lg[None], [max_pos - 5], text[None], pad, params, [1])
    assert e.value.status == qtts.QTTS_ERANGE
    with pytest.raises(qtts.QttsError) as e:
        t.forward_with_embedding(lh, kv, max_pos)
    assert e.value.status == qtts.QTTS_ERANGE
    # a cache too small for max_codes more rows
    small = t.new_kv(9)
    with pytest.raises(qtts.QttsError) as e:
        qtts.generate_codes(t, p, small, p.new_kv(), lh, lg, 0, text, pad, params, seed=1)
    assert e.value.status == qtts.QTTS_ERANGE
    with pytest.raises(qtts.QttsError) as e:
        qtts.generate_codes_batch(t, p, [small], lh[None], lg[None], [0], text[None], pad, params, [1])
    assert e.value.status == qtts.QTTS_ERANGE
    # a full cache refuses one more decode step
    one = t.new_kv(1)
    t.forward_with_embedding(lh, one, 0)
    with pytest.raises(qtts.QttsError) as e:
        t.forward_with_embedding(lh, one, 1)
    assert e.value.status == qtts.QTTS_ERANGE
    assert len(kv) == len(small) == 0 and len(one) == 1
    _clean_loop_matches(tiny, 78)
