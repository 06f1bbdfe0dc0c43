"""GPU parity of the batched loop (qtts_generate_codes_batch): several
independent streams in lockstep -- each with its own prompt, cache, position,
trailing text and seed -- give, stream by stream, the codes the oracle's
single-stream loop gives (greedy and sampled, with and without the code
predictor), and the caches are left where single-stream loops leave them."""
import numpy as np
import pytest

import qtts
from oracle import oracle
from shapes import FULL_PREDICTOR, FULL_TALKER, TINY_PREDICTOR, TINY_TALKER, rel_err, within

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def tiny(ctx):
    tw = qtts.TalkerWeights(61, TINY_TALKER)
    pw = qtts.CodePredictorWeights(61, TINY_PREDICTOR, talker_hidden=TINY_TALKER.hidden)
    return (tw, pw, qtts.Talker(ctx, tw), qtts.CodePredictor(ctx, pw), oracle.Talker(tw, nthreads=1),
            oracle.CodePredictor(pw, nthreads=1))


def _streams(tw, t, ot, B, seed, prompt_lens, cap, trailing=3):
    """Prefilled caches (GPU and oracle) and the loop inputs of B streams."""
    H = tw.cfg.hidden
    kvs, okvs, lhs, lgs, pos = [], [], [], [], []
    for b in range(B):
        n = prompt_lens[b]
        x = qtts.synth_normal_f32(seed, f"batch.prompt.{b}", n * H)
        kv, okv = t.new_kv(cap), ot.new_kv(cap)
        t.prefill_talker_raw(x, n, kv)
        lh = ot.prefill_talker_raw(x, n, okv)
        kvs.append(kv)
        okvs.append(okv)
        lhs.append(lh)
        lgs.append(ot.apply_codec_head(lh))
        pos.append(n)
    text = qtts.synth_normal_f32(seed, "batch.text", B * trailing * H, 0.0, 0.1).reshape(B, trailing, H)
    pad = qtts.synth_normal_f32(seed, "batch.pad", H, 0.0, 0.1)
    return kvs, okvs, np.stack(lhs), np.stack(lgs), pos, text, pad


@pytest.mark.parametrize("greedy", [True, False])
def test_batch_matches_oracle_streams(tiny, greedy):
    tw, pw, t, p, ot, op = tiny
    B, frames = 5, 24
    lens = [10, 6, 13, 10, 9]
    kvs, okvs, lh, lg, pos, text, pad = _streams(tw, t, ot, B, 62, lens, 64)
    seeds = [1000 + 17 * b for b in range(B)]
    params = qtts.loop_params(frames, greedy=greedy, stop_on_eos=False)
    got = qtts.generate_codes_batch(t, p, kvs, lh, lg, pos, text, pad, params, seeds)
    for b in range(B):
        ref = oracle.generate_codes(ot, op, okvs[b], op.new_kv(), lh[b], lg[b], pos[b], text[b], pad, params,
                                    seed=seeds[b])
        assert got[b].shape == ref.shape == (16, frames)
        assert np.array_equal(got[b], ref), (b, np.argwhere(got[b] != ref)[:5])
        assert len(kvs[b]) == lens[b] + frames
        # the rows the loop appended (QK-normed, rotated K and raw V, written
        # by the attention kernel itself) match the oracle's cache
        (gk, gv), (rk, rv) = kvs[b].store(), okvs[b].store()
        assert gk.shape == rk.shape
        assert within(gk, rk) and within(gv, rv), b


@pytest.mark.parametrize("B", [1, 20, 64])
def test_batch_sizes(tiny, B):
    """One stream, more streams than one 16-row tile (the first pass's 2B
    rows then span two or more 32-row matrix-core tiles: 40 rows, and 128
    rows in two 64-row chunks at the 64-stream maximum): sampled codes and
    caches match the oracle's single-stream loops."""
    tw, pw, t, p, ot, op = tiny
    frames = 4
    lens = [5 + (7 * b) % 10 for b in range(B)]
    kvs, okvs, lh, lg, pos, text, pad = _streams(tw, t, ot, B, 67, lens, 24, trailing=2)
    seeds = [3000 + 11 * b for b in range(B)]
    params = qtts.loop_params(frames, temperature=0.8, top_k=50, repetition_penalty=1.05, stop_on_eos=False)
    got = qtts.generate_codes_batch(t, p, kvs, lh, lg, pos, text, pad, params, seeds)
    assert len(got) == B
    for b in range(B):
        ref = oracle.generate_codes(ot, op, okvs[b], op.new_kv(), lh[b], lg[b], pos[b], text[b], pad, params,
                                    seed=seeds[b])
        assert got[b].shape == ref.shape == (16, frames)
        assert np.array_equal(got[b], ref), (b, np.argwhere(got[b] != ref)[:5])
        (gk, gv), (rk, rv) = kvs[b].store(), okvs[b].store()
        assert gk.shape == rk.shape
        assert within(gk, rk) and within(gv, rv), b
    for kv in kvs:
        kv.close()


def test_batch_is_deterministic(tiny):
    """The same 5-stream batch twice with the same seeds and inputs: every
    stream's codes and cache are identical bit for bit."""
    tw, pw, t, p, ot, op = tiny
    B, frames = 5, 16
    lens = [10, 6, 13, 10, 9]
    seeds = [2000 + 5 * b for b in range(B)]
    params = qtts.loop_params(frames, temperature=0.8, top_k=50, repetition_penalty=1.05, stop_on_eos=False)
    runs = []
    for _ in range(2):
        kvs, _okvs, lh, lg, pos, text, pad = _streams(tw, t, ot, B, 63, lens, 48)
        codes = qtts.generate_codes_batch(t, p, kvs, lh, lg, pos, text, pad, params, seeds)
        runs.append((codes, [kv.store() for kv in kvs]))
        for kv in kvs:
            kv.close()
    (c0, s0), (c1, s1) = runs
    for b in range(B):
        assert np.array_equal(c0[b], c1[b]), b
        assert np.array_equal(s0[b][0], s1[b][0]) and np.array_equal(s0[b][1], s1[b][1]), b


def test_batch_long_caches(tiny):
    """Streams deep into long caches (700-900 prompt rows of a 1000-row
    capacity): every talker attention split spans dozens of positions and
    the new row lands in the last one, which appends it; codes and caches
    match the oracle's."""
    tw, pw, t, p, ot, op = tiny
    B, frames = 2, 4
    lens = [700, 900]
    kvs, okvs, lh, lg, pos, text, pad = _streams(tw, t, ot, B, 65, lens, 1000)
    params = qtts.loop_params(frames, greedy=True, stop_on_eos=False)
    got = qtts.generate_codes_batch(t, p, kvs, lh, lg, pos, text, pad, params, [3, 4])
    for b in range(B):
        ref = oracle.generate_codes(ot, op, okvs[b], op.new_kv(), lh[b], lg[b], pos[b], text[b], pad, params, seed=3 + b)
        assert np.array_equal(got[b], ref), (b, np.argwhere(got[b] != ref)[:5])
        (gk, gv), (rk, rv) = kvs[b].store(), okvs[b].store()
        assert gk.shape == rk.shape
        assert within(gk, rk) and within(gv, rv), b


def test_batch_talker_only_and_eos(tiny):
    """Talker-only loops; with EOS on, each stream stops on its own frame."""
    tw, _, t, _, ot, _ = tiny
    B, frames = 3, 20
    kvs, okvs, lh, lg, pos, _, _ = _streams(tw, t, ot, B, 63, [8, 8, 8], 32)
    params = qtts.loop_params(frames, greedy=True, stop_on_eos=False, talker_only=True)
    got = qtts.generate_codes_batch(t, None, kvs, lh, lg, pos, None, None, params, [5, 6, 7])
    refs = []
    for b in range(B):
        ref = oracle.generate_codes(ot, None, okvs[b], None, lh[b], lg[b], pos[b], None, None, params, seed=5 + b)
        assert np.array_equal(got[b], ref)
        refs.append(ref)
    # make stream 1's 4th code EOS: stream 1 stops before that frame, the others run on
    eos = int(refs[1][0, 3])
    params = qtts.loop_params(frames, greedy=True, stop_on_eos=True, talker_only=True, codec_eos_id=eos)
    kvs, okvs, lh, lg, pos, _, _ = _streams(tw, t, ot, B, 63, [8, 8, 8], 32)
    got = qtts.generate_codes_batch(t, None, kvs, lh, lg, pos, None, None, params, [5, 6, 7])
    for b in range(B):
        ref = oracle.generate_codes(ot, None, okvs[b], None, lh[b], lg[b], pos[b], None, None, params, seed=5 + b)
        assert got[b].shape == ref.shape and np.array_equal(got[b], ref), b
    assert got[1].shape[1] == int(np.argmax(refs[1][0] == eos))


def test_batch_full_model(ctx):
    """The 1.7B talker and predictor, 4 streams x 3 sampled frames."""
    tw = qtts.TalkerWeights(1, FULL_TALKER)
    pw = qtts.CodePredictorWeights(1, FULL_PREDICTOR, talker_hidden=FULL_TALKER.hidden)
    t, p = qtts.Talker(ctx, tw), qtts.CodePredictor(ctx, pw)
    ot, op = oracle.Talker(tw), oracle.CodePredictor(pw)
    B, frames = 4, 3
    kvs, okvs, lh, lg, pos, text, pad = _streams(tw, t, ot, B, 64, [12, 12, 12, 12], 32, trailing=2)
    params = qtts.loop_params(frames, temperature=0.8, top_k=50, repetition_penalty=1.05, stop_on_eos=False)
    got = qtts.generate_codes_batch(t, p, kvs, lh, lg, pos, text, pad, params, [31, 32, 33, 34])
    for b in range(B):
        ref = oracle.generate_codes(ot, op, okvs[b], op.new_kv(), lh[b], lg[b], pos[b], text[b], pad, params,
                                    seed=31 + b)
        assert np.array_equal(got[b], ref), (b, np.argwhere(got[b] != ref)[:5])


def test_batch_without_predictor_tables(ctx, tiny, monkeypatch):
    """QTTS_PREDICTOR_TABLE=0 (read when a predictor first runs): passes
    2-15 of the batched loop gather the previous code's embedding and run the
    input projection as a GEMM of their own instead of reading the per-code
    table.  Codes still match the oracle's single-stream loops."""
    tw, pw, t, _, ot, op = tiny
    monkeypatch.setenv("QTTS_PREDICTOR_TABLE", "0")
    p_off = qtts.CodePredictor(ctx, pw)
    B, frames = 3, 8
    kvs, okvs, lh, lg, pos, text, pad = _streams(tw, t, ot, B, 66, [9, 12, 7], 32)
    params = qtts.loop_params(frames, temperature=0.8, top_k=50, repetition_penalty=1.05, stop_on_eos=False)
    got = qtts.generate_codes_batch(t, p_off, kvs, lh, lg, pos, text, pad, params, [41, 42, 43])
    for b in range(B):
        ref = oracle.generate_codes(ot, op, okvs[b], op.new_kv(), lh[b], lg[b], pos[b], text[b], pad, params,
                                    seed=41 + b)
        assert np.array_equal(got[b], ref), (b, np.argwhere(got[b] != ref)[:5])
