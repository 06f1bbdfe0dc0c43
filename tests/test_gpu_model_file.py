"""GPU tests of a model loaded from a .qora-tts file: the talker and the
code predictor uploaded from the file's views (with the file's RoPE tables)
give the same bits as the same weights uploaded from memory, and the sampled
frame loop over them matches the oracle run on the file, code for code."""
import numpy as np
import pytest

import qtts
from oracle import oracle
from qtts_file_writer import TextWeights, write_model
from shapes import TINY_PREDICTOR, TINY_TALKER

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def loaded(ctx, tmp_path_factory):
    tw = qtts.TalkerWeights(43, TINY_TALKER)
    pw = qtts.CodePredictorWeights(43, TINY_PREDICTOR, talker_hidden=TINY_TALKER.hidden)
    text = TextWeights(43, text_vocab=96, text_hidden=64, hidden=TINY_TALKER.hidden)
    trope = oracle.build_rope_table(TINY_TALKER.head_dim, TINY_TALKER.max_position, TINY_TALKER.rope_theta)
    prope = oracle.build_rope_table(TINY_PREDICTOR.head_dim, 64, TINY_PREDICTOR.rope_theta)
    path = str(tmp_path_factory.mktemp("model") / "tiny.qora-tts")
    write_model(path, tw, pw, text, trope, prope)
    f = qtts.ModelFile(path)
    return tw, pw, f


def test_file_upload_matches_memory_upload(ctx, loaded):
    tw, pw, f = loaded
    tf, tm = qtts.Talker(ctx, f.talker), qtts.Talker(ctx, tw)
    kvf, kvm = tf.new_kv(16), tm.new_kv(16)
    x = qtts.synth_normal_f32(44, "mf.prefill", 9 * TINY_TALKER.hidden)
    assert np.array_equal(tf.prefill_talker_raw(x, 9, kvf), tm.prefill_talker_raw(x, 9, kvm))
    for pos in range(9, 12):
        emb = qtts.synth_normal_f32(44, f"mf.emb.{pos}", TINY_TALKER.hidden)
        assert np.array_equal(tf.forward_with_embedding(emb, kvf, pos), tm.forward_with_embedding(emb, kvm, pos))
    pf, pm = qtts.CodePredictor(ctx, f.predictor), qtts.CodePredictor(ctx, pw)
    h = qtts.synth_normal_f32(44, "mf.h", TINY_TALKER.hidden)
    s = qtts.synth_normal_f32(44, "mf.s", TINY_TALKER.hidden)
    assert np.array_equal(pf.generate_acoustic_codes(h, s, pf.new_kv()), pm.generate_acoustic_codes(h, s, pm.new_kv()))


def test_file_loop_matches_oracle(ctx, loaded):
    _, _, f = loaded
    t, p = qtts.Talker(ctx, f.talker), qtts.CodePredictor(ctx, f.predictor)
    ot, op = oracle.Talker(f.talker), oracle.CodePredictor(f.predictor)
    hidden = TINY_TALKER.hidden
    text = qtts.synth_normal_f32(45, "mf.text", 3 * hidden, 0.0, 0.1).reshape(3, hidden)
    pad = qtts.synth_normal_f32(45, "mf.pad", hidden, 0.0, 0.1)
    x = qtts.synth_normal_f32(45, "mf.loop.prefill", 10 * hidden)
    kv, okv = t.new_kv(64), ot.new_kv(64)
    t.prefill_talker_raw(x, 10, kv)
    olh = ot.prefill_talker_raw(x, 10, okv)
    logits = ot.apply_codec_head(olh)
    params = qtts.loop_params(32, greedy=False, stop_on_eos=False)
    got = qtts.generate_codes(t, p, kv, p.new_kv(), olh, logits, 10, text, pad, params, seed=99)
    ref = oracle.generate_codes(ot, op, okv, op.new_kv(), olh, logits, 10, text, pad, params, seed=99)
    assert np.array_equal(got, ref), np.argwhere(got != ref)[:5]
