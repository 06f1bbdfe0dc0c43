"""GPU path against the committed known-answer vectors (tests/golden): the
small Q4 GEMV, the small talker's decode steps and prefill, and the small
predictor's codes, all from the float64 model, not from the oracle."""
import os

import numpy as np
import pytest

import qtts
from shapes import TINY_PREDICTOR, TINY_TALKER, rel_err, within

pytestmark = pytest.mark.gpu
GOLDEN = np.load(os.path.join(os.path.dirname(__file__), "golden", "golden.npz"))
REL_TOL = 1e-3


def test_gemv_golden(ctx):
    w = qtts.Q4Weight(GOLDEN["gemv_packed"], GOLDEN["gemv_scales"], 64, 96)
    y = qtts.DeviceQ4(ctx, w).gemv(GOLDEN["gemv_x"])
    assert rel_err(y, GOLDEN["gemv_y"]) < 1e-6


def test_talker_and_predictor_golden(ctx):
    H = TINY_TALKER.hidden
    tw = qtts.TalkerWeights(31, TINY_TALKER)
    pw = qtts.CodePredictorWeights(31, TINY_PREDICTOR, talker_hidden=H)
    t, p = qtts.Talker(ctx, tw), qtts.CodePredictor(ctx, pw)
    kv = t.new_kv(8)
    s0 = t.forward_with_embedding(qtts.synth_normal_f32(31, "golden.emb", H), kv, 0)
    s1 = t.forward_with_embedding(qtts.synth_normal_f32(31, "golden.emb1", H), kv, 1)
    assert within(s0, GOLDEN["talker_step0"])
    assert within(s1, GOLDEN["talker_step1"])
    X = qtts.synth_normal_f32(31, "golden.prefill", 6 * H)
    assert rel_err(t.prefill_talker_raw(X, 6, t.new_kv(8)), GOLDEN["talker_prefill6"]) < REL_TOL
    h = GOLDEN["talker_step0"][:H].astype(np.float32)
    codes = p.generate_acoustic_codes(h, t.embed_codec_token(11), p.new_kv())
    assert np.array_equal(codes, GOLDEN["pred_codes"])
