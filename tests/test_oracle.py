"""CPU tests that pin the oracle (what the parity tests compare with) and the library's host
logic.  Each check is chosen so that a plausible mistake fails it: closed
forms (binary16, xorshift, RoPE, RMSNorm of a constant), invariants (one-hot
GEMV, thread-split invariance, prefill == sequential decode, RoPE norm
preservation), float64 brute force (GEMV, the numpy model of the talker step
and predictor frame), and hand-built sampler cases for each ordering rule of
sample_token (src/generate_new.rs:329-391).
"""
import os

import numpy as np
import pytest

import qtts
from oracle import oracle
from shapes import GEMV_SHAPES, TINY_PREDICTOR, TINY_TALKER, rel_err
import numpy_model as nm

GOLDEN = np.load(os.path.join(os.path.dirname(__file__), "golden", "golden.npz"))
MASK = (1 << 64) - 1


# ---------------------------------------------------------------- binary16
def test_f16_to_f32_every_pattern():
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    ref = bits.view(np.float16).astype(np.float32)
    lib = qtts.load_library()
    got_o = np.array([oracle.f16_to_f32(int(b)) for b in bits], dtype=np.float32)
    got_l = np.array([lib.qtts_f16_to_f32(int(b)) for b in bits], dtype=np.float32)
    nan = np.isnan(ref)
    for got in (got_o, got_l):
        assert np.array_equal(np.isnan(got), nan)
        assert np.array_equal(got[~nan].view(np.uint32), ref[~nan].view(np.uint32))


def test_f32_to_f16_round_to_nearest_even():
    lib = qtts.load_library()
    vals = GOLDEN["f16_in"].view(np.float32)
    got = np.array([lib.qtts_f32_to_f16(float(v)) for v in vals], dtype=np.uint16)
    assert np.array_equal(got, GOLDEN["f16_out"])


# ---------------------------------------------------------------- xorshift
def test_simple_rand_known_answers():
    for seed, states, rs in zip(GOLDEN["xs_seeds"], GOLDEN["xs_states"], GOLDEN["xs_r"]):
        st = int(seed)
        for s_ref, r_ref in zip(states, rs):
            r, st = oracle.simple_rand(st)
            assert st == int(s_ref)
            assert np.float32(r).view(np.uint32) == np.float32(r_ref).view(np.uint32)


def test_simple_rand_can_return_one():
    """f32(state) rounds to 2^64 for the top 2^39 states: r == 1.0 exactly."""
    r, _ = oracle.simple_rand(_preimage(MASK))
    assert r == 1.0


def _unshift_left(y, k):
    x = y
    for _ in range(64 // k + 1):
        x = y ^ ((x << k) & MASK)
    return x


def _unshift_right(y, k):
    x = y
    for _ in range(64 // k + 1):
        x = y ^ (x >> k)
    return x


def _preimage(target):
    """State s with xorshift(s) == target (xorshift64 is a bijection)."""
    x = _unshift_left(target, 17)
    x = _unshift_right(x, 7)
    return _unshift_left(x, 13)


def test_xorshift_preimage_helper():
    for t in (1, 12345, MASK, 0x8000000000000001):
        s = _preimage(t)
        s2 = s ^ ((s << 13) & MASK)
        s2 ^= s2 >> 7
        s2 ^= (s2 << 17) & MASK
        assert s2 == t


# ---------------------------------------------------------------- Q4 + GEMV
def test_dequant_known_bytes():
    """0x00 -> (-8,-8)*s, 0x8F -> (7,0)*s, 0xF8 -> (0,7)*s (low nibble = even column)."""
    packed = np.zeros((2, 16), dtype=np.uint8)
    packed[0, :3] = [0x00, 0x8F, 0xF8]
    packed[1, 0] = 0x8F
    scales = np.array([[0x3C00], [0x3800]], dtype=np.uint16)  # 1.0, 0.5
    w = qtts.Q4Weight(packed, scales, 2, 32)
    r0 = oracle.embed_lookup(w, 0)
    assert r0[:6].tolist() == [-8.0, -8.0, 7.0, 0.0, 0.0, 7.0]
    assert np.all(r0[6:] == -8.0)
    assert oracle.embed_lookup(w, 1)[:2].tolist() == [3.5, 0.0]


def test_gemv_golden_small():
    w = qtts.Q4Weight(GOLDEN["gemv_packed"], GOLDEN["gemv_scales"], 64, 96)
    y = oracle.gemv(GOLDEN["gemv_x"], w, 1)
    assert rel_err(y, GOLDEN["gemv_y"]) < 1e-6


@pytest.mark.parametrize("K,N", GEMV_SHAPES)
@pytest.mark.parametrize("nthreads", [1, 8])
def test_gemv_config1_vs_float64(K, N, nthreads):
    w = qtts.Q4Weight.synthetic(11, f"gemv.{K}x{N}", K, N)
    x = qtts.synth_normal_f32(11, f"gemv.x.{K}", K)
    y = oracle.gemv(x, w, nthreads)
    exact = w.dequantize().astype(np.float64).T @ x.astype(np.float64)
    assert rel_err(y, exact) < 1e-5


def test_gemv_one_hot_is_exact_row():
    w = qtts.Q4Weight.synthetic(12, "onehot", 2048, 4096)
    w.scales[3, :4] = [1, 0x3FF, 0, 0x200]  # binary16 subnormals and a zero scale
    deq = w.dequantize()
    for k in (0, 3, 2047):
        x = np.zeros(2048, dtype=np.float32)
        x[k] = 1.0
        assert np.array_equal(oracle.gemv(x, w, 8), deq[k])


def test_gemv_thread_split_invariance():
    """Split-K over 1, 3, 8, 16 threads changes only rounding."""
    w = qtts.Q4Weight.synthetic(13, "split", 6144, 2048)
    x = qtts.synth_normal_f32(13, "split.x", 6144)
    ys = [oracle.gemv(x, w, t) for t in (1, 3, 8, 16)]
    for y in ys[1:]:
        assert rel_err(y, ys[0]) < 1e-5


def test_gemv_small_matrices_ignore_threads():
    """k*n < 4e6 runs single-threaded (src/gemv.rs:268-272): bitwise equal."""
    w = qtts.Q4Weight.synthetic(14, "small", 1024, 3072)
    x = qtts.synth_normal_f32(14, "small.x", 1024)
    assert np.array_equal(oracle.gemv(x, w, 1).view(np.uint32), oracle.gemv(x, w, 16).view(np.uint32))


def test_gemv_zero_input_and_zero_scale_rows_skipped():
    w = qtts.Q4Weight.synthetic(15, "zeros", 256, 128)
    x = qtts.synth_normal_f32(15, "zeros.x", 256)
    x[:100] = 0.0
    w.scales[100:140] = 0
    exact = w.dequantize().astype(np.float64).T @ x.astype(np.float64)
    assert rel_err(oracle.gemv(x, w, 1), exact) < 1e-6


def test_gemm_rows_equal_gemv():
    w = qtts.Q4Weight.synthetic(16, "gemm", 2048, 2048)
    x = qtts.synth_normal_f32(16, "gemm.x", 5 * 2048)
    y = oracle.gemm(x, 5, w, 8).reshape(5, 2048)
    for t in range(5):
        assert np.array_equal(y[t], oracle.gemv(x[t * 2048:(t + 1) * 2048], w, 1))


def test_quantizer_rules():
    """quantize_f32_to_q4: scale = absmax/7 as binary16; q = round half away
    from zero of v/scale (float32 scale), clamped; dequant error <= scale/2."""
    rng = np.random.default_rng(5)
    data = (rng.standard_normal((8, 64)) * 0.05).astype(np.float32)
    data[0, :32] = 0.0  # all-zero group
    data[1, 0] = 0.35   # exact multiple of absmax/7 boundary cases
    w = qtts.Q4Weight.quantize(data)
    g = data.reshape(8, 2, 32)
    scale32 = np.abs(g).max(axis=2) / np.float32(7.0)
    assert np.array_equal(w.scales, scale32.astype(np.float16).view(np.uint16))
    with np.errstate(divide="ignore"):
        inv = np.where(scale32 > 0, np.float32(1.0) / scale32, np.float32(0.0)).astype(np.float32)
    v = (g * inv[:, :, None]).astype(np.float32)
    q = np.clip(np.sign(v) * np.floor(np.abs(v) + np.float32(0.5)), -8, 7).astype(np.int32)
    assert np.array_equal(w.nibbles().reshape(8, 2, 32), (q + 8).astype(np.uint8))
    s16 = w.scales.view(np.float16).astype(np.float32)
    assert np.all(np.abs(w.dequantize().reshape(8, 2, 32) - g) <= s16[:, :, None] * 0.5 + 1e-3 * s16[:, :, None])


# ---------------------------------------------------------------- norms etc
def test_rms_norm_closed_form_and_float64():
    g1 = np.full(2048, 0x3C00, dtype=np.uint16)
    c = np.float32(0.75)
    y = oracle.rms_norm_f16(np.full(2048, c, dtype=np.float32), g1)
    assert np.allclose(y, c / np.sqrt(c * c + 1e-6), rtol=2e-7)
    x = qtts.synth_normal_f32(1, "rms.x", 2048)
    g = qtts.synth_normal_f16(1, "rms.g", 2048)
    assert rel_err(oracle.rms_norm_f16(x, g), nm.rms_norm(x, g)) < 1e-6


def test_qk_norm_per_head_shared_gamma():
    x = qtts.synth_normal_f32(2, "qk.x", 16 * 128)
    g = qtts.synth_normal_f16(2, "qk.g", 128)
    ref = nm.rms_norm(x.reshape(16, 128), g).reshape(-1)
    assert rel_err(oracle.qk_norm(x, 16, 128, g), ref) < 1e-6


def test_softmax_raw():
    s = qtts.synth_normal_f32(3, "sm", 600, 0.0, 5.0)
    p = oracle.softmax_raw(s)
    e = np.exp(s.astype(np.float64) - s.max())
    assert rel_err(p, e / e.sum()) < 1e-6
    assert abs(p.astype(np.float64).sum() - 1.0) < 1e-5
    assert np.array_equal(oracle.softmax_raw(s + np.float32(3.0)).argmax(), p.argmax())


def test_silu_closed_form():
    for v in (-20.0, -1.5, -1e-3, 0.0, 0.5, 3.0, 30.0):
        assert abs(oracle.silu(v) - v / (1 + np.exp(-v))) <= 1e-6 * max(1.0, abs(v))


# ---------------------------------------------------------------- RoPE
def test_rope_table_entries():
    cos_t, sin_t = oracle.build_rope_table(128, 32768, 1.0e6)
    for a, p in enumerate(GOLDEN["rope_pos"]):
        for b, i in enumerate(GOLDEN["rope_i"]):
            # float64 cos/sin rounded once to float32: libm and numpy agree
            # to well under half an ulp, so the float32 values are identical
            assert cos_t[p, i] == GOLDEN["rope_cos"][a, b]
            assert sin_t[p, i] == GOLDEN["rope_sin"][a, b]
    assert np.all(cos_t[0] == 1.0) and np.all(sin_t[0] == 0.0)


def test_rope_split_pairs_and_norms():
    cos_t, sin_t = oracle.build_rope_table(128, 600, 1.0e6)
    x = qtts.synth_normal_f32(4, "rope.x", 4 * 128)
    assert np.array_equal(oracle.rope_split(x, 4, 128, 0, cos_t, sin_t), x)
    y = oracle.rope_split(x, 4, 128, 563, cos_t, sin_t).reshape(4, 128)
    ref = nm.rope(x.reshape(4, 128).astype(np.float64), 563, 1.0e6)
    assert rel_err(y, ref) < 1e-6
    xr = x.reshape(4, 128)
    n0 = xr[:, :64] ** 2 + xr[:, 64:] ** 2
    n1 = y[:, :64].astype(np.float64) ** 2 + y[:, 64:].astype(np.float64) ** 2
    assert np.allclose(n0, n1, rtol=1e-5, atol=1e-6)


# ---------------------------------------------------------------- composites
@pytest.fixture(scope="module")
def tiny():
    tw = qtts.TalkerWeights(31, TINY_TALKER)
    pw = qtts.CodePredictorWeights(31, TINY_PREDICTOR, talker_hidden=TINY_TALKER.hidden)
    return tw, pw, oracle.Talker(tw, 1), oracle.CodePredictor(pw, 1)


def test_synthetic_generator_pins():
    lib = qtts.load_library()
    assert [lib.qtts_synth_u64(7, 11, i) for i in range(8)] == [int(v) for v in GOLDEN["synth_u64"]]
    sw = qtts.Q4Weight.synthetic(3, "golden.synth", 32, 64)
    assert np.array_equal(sw.packed[:2], GOLDEN["synth_packed"])
    assert np.array_equal(sw.scales[:4], GOLDEN["synth_scales"])
    assert np.array_equal(qtts.synth_normal_f32(3, "golden.normal", 16), GOLDEN["synth_normal"])


def test_talker_steps_vs_float64_model(tiny):
    tw, _, ot, _ = tiny
    kv = ot.new_kv(8)
    emb = qtts.synth_normal_f32(31, "golden.emb", TINY_TALKER.hidden)
    emb1 = qtts.synth_normal_f32(31, "golden.emb1", TINY_TALKER.hidden)
    assert rel_err(ot.forward_with_embedding(emb, kv, 0), GOLDEN["talker_step0"]) < 1e-5
    assert rel_err(ot.forward_with_embedding(emb1, kv, 1), GOLDEN["talker_step1"]) < 1e-5


def test_talker_prefill_vs_float64_model(tiny):
    tw, _, ot, _ = tiny
    X = qtts.synth_normal_f32(31, "golden.prefill", 6 * TINY_TALKER.hidden)
    assert rel_err(ot.prefill_talker_raw(X, 6, ot.new_kv(8)), GOLDEN["talker_prefill6"]) < 1e-5


def test_prefill_equals_sequential_decode(tiny):
    """prefill_talker_raw(S tokens) == S forward steps at positions 0..S-1:
    same cache, same final hidden (different code paths in the oracle)."""
    tw, _, ot, _ = tiny
    S, H = 7, TINY_TALKER.hidden
    X = qtts.synth_normal_f32(32, "seq", S * H)
    kv1, kv2 = ot.new_kv(S), ot.new_kv(S)
    h1 = ot.prefill_talker_raw(X, S, kv1)
    for t in range(S):
        h2 = ot.forward_with_embedding(X[t * H:(t + 1) * H], kv2, t)[:H]
    assert rel_err(h1, h2) < 1e-5
    (k1, v1), (k2, v2) = kv1.store(), kv2.store()
    assert rel_err(k1, k2) < 1e-5 and rel_err(v1, v2) < 1e-5


def test_predictor_vs_float64_model(tiny):
    tw, pw, ot, op = tiny
    h = GOLDEN["talker_step0"][: TINY_TALKER.hidden].astype(np.float32)
    sem = ot.embed_codec_token(11)
    codes = op.generate_acoustic_codes(h, sem, op.new_kv())
    assert np.array_equal(codes, GOLDEN["pred_codes"])


def test_acoustic_embedding_sum(tiny):
    _, pw, _, op = tiny
    codes = np.arange(15, dtype=np.uint32) * 13 % TINY_PREDICTOR.vocab
    ref = np.zeros(TINY_TALKER.hidden, dtype=np.float32)
    for g, c in enumerate(codes):
        ref += pw.codec_embeddings[g].dequantize()[c]
    assert np.array_equal(op.get_acoustic_embeddings_sum(codes), ref)


def test_kv_roundtrip():
    kv = oracle.Kv(3, 2, 128, 10)
    k = qtts.synth_normal_f32(6, "kv.k", 3 * 7 * 2 * 128).reshape(3, 7, 2, 128)
    v = qtts.synth_normal_f32(6, "kv.v", 3 * 7 * 2 * 128).reshape(3, 7, 2, 128)
    kv.load(k, v, 7)
    k2, v2 = kv.store()
    assert np.array_equal(k, k2) and np.array_equal(v, v2) and len(kv) == 7


# ---------------------------------------------------------------- sampler
def _seed_for_r(lo, hi):
    """A seed whose first simple_rand draw falls in [lo, hi)."""
    for i in range(1, 100000):
        s = (i * 0x9E3779B97F4A7C15) & MASK  # well-mixed candidates
        r, _ = oracle.simple_rand(s)
        if lo <= r < hi:
            return s
    raise AssertionError("no seed found")


def test_sampler_cumsum_in_index_order():
    """p = [0.25, 0.75]: r = 0.2 picks index 0 in index order (a sorted-order
    cumsum would pick 1)."""
    logits = np.array([0.0, np.log(3.0)], dtype=np.float32)
    seed = _seed_for_r(0.05, 0.24)
    assert oracle.sample_token(logits, 1.0, 0, 1.0, (), seed)[0] == 0
    seed = _seed_for_r(0.26, 0.99)
    assert oracle.sample_token(logits, 1.0, 0, 1.0, (), seed)[0] == 1


def test_sampler_topk_ties_keep_lower_indices():
    """Stable descending sort: of three equal maxima, top_k=2 keeps the two
    lowest indices, each at p = 0.5."""
    logits = np.array([1.0, 3.0, 3.0, 3.0, 0.0], dtype=np.float32)
    assert oracle.sample_token(logits, 1.0, 2, 1.0, (), _seed_for_r(0.0, 0.49))[0] == 1
    assert oracle.sample_token(logits, 1.0, 2, 1.0, (), _seed_for_r(0.51, 0.99))[0] == 2


def test_sampler_top1_and_fallback_zero():
    logits = qtts.synth_normal_f32(7, "top1", 3072, 0.0, 3.0)
    best = int(np.argmax(logits))
    assert oracle.sample_token(logits, 0.8, 1, 1.0, (), 99)[0] == best
    # r == 1.0 is never < the final cumsum (1.0): fallback token 0
    tok, _ = oracle.sample_token(logits, 0.8, 1, 1.0, (), _preimage(MASK))
    assert tok == 0


def test_sampler_penalty_applies_per_entry():
    """prev_tokens entries penalise once each, duplicates included; positive
    logits divide, others multiply (src/generate_new.rs:333-343)."""
    logits = np.array([2.0, -2.0, 1.9, -10.0], dtype=np.float32)
    # greedy mode exposes the penalised argmax: 2/1.05^2 = 1.814 < 1.9
    assert oracle.sample_token(logits, 1.0, 0, 1.05, (0, 0), 1, greedy=True)[0] == 2
    assert oracle.sample_token(logits, 1.0, 0, 1.05, (0,), 1, greedy=True)[0] == 0
    # -2 * 1.05^16 = -4.37 still > -10; the penalised entry is never picked
    assert oracle.sample_token(logits[[1, 3]], 1.0, 0, 1.05, (0,) * 16, 1, greedy=True)[0] == 0


def test_sampler_greedy_last_max_and_nan():
    logits = np.zeros(8, dtype=np.float32)
    logits[[2, 5]] = 1.0
    assert oracle.sample_token(logits, 1.0, 0, 1.0, (), 1, greedy=True)[0] == 5
    assert oracle.argmax(logits) == 5
    logits[3] = np.nan
    with pytest.raises(oracle.OracleError):
        oracle.argmax(logits)
    with pytest.raises(oracle.OracleError):
        oracle.sample_token(logits, 0.8, 3, 1.0, (), 1)


def test_sampler_distribution_matches_probabilities():
    """Frequencies over many seeds follow the top-k renormalised softmax."""
    logits = np.array([0.0, 1.0, 2.0, 0.5, -1.0], dtype=np.float32)
    counts = np.zeros(5)
    st = 12345
    for _ in range(4000):
        tok, st = oracle.sample_token(logits, 0.8, 3, 1.0, (), st)
        counts[tok] += 1
    p = np.exp(logits / 0.8)
    p[np.argsort(-p)[3:]] = 0
    p /= p.sum()
    assert np.all(np.abs(counts / 4000 - p) < 0.03)


# ---------------------------------------------------------------- loop
def test_loop_eos_stops_before_frame(tiny):
    tw, pw, ot, op = tiny
    H = TINY_TALKER.hidden
    lh = GOLDEN["talker_step0"][:H].astype(np.float32)
    logits = GOLDEN["talker_step0"][H:].astype(np.float32)
    text = qtts.synth_normal_f32(8, "t", 2 * H, 0, 0.1).reshape(2, H)
    pad = qtts.synth_normal_f32(8, "p", H, 0, 0.1)
    p0 = qtts.loop_params(12, greedy=False, stop_on_eos=False)
    ref = oracle.generate_codes(ot, op, ot.new_kv(16), op.new_kv(), lh, logits, 0, text, pad, p0, seed=5)
    assert ref.shape == (16, 12)
    eos = int(ref[0, 4])
    first = int(np.argmax(ref[0] == eos))
    p1 = qtts.loop_params(12, greedy=False, stop_on_eos=True, codec_eos_id=eos)
    kv = ot.new_kv(16)
    got = oracle.generate_codes(ot, op, kv, op.new_kv(), lh, logits, 0, text, pad, p1, seed=5)
    assert got.shape == (16, first) and np.array_equal(got, ref[:, :first]) and len(kv) == first


def test_loop_frame_matches_manual_composition(tiny):
    """One frame of the loop == sample_token -> generate_acoustic_codes ->
    embedding sum + text -> forward_with_embedding, composed by hand."""
    tw, pw, ot, op = tiny
    H = TINY_TALKER.hidden
    lh = GOLDEN["talker_step0"][:H].astype(np.float32)
    logits = GOLDEN["talker_step0"][H:].astype(np.float32)
    text = qtts.synth_normal_f32(9, "t", H, 0, 0.1).reshape(1, H)
    pad = qtts.synth_normal_f32(9, "p", H, 0, 0.1)
    codes = oracle.generate_codes(ot, op, ot.new_kv(4), op.new_kv(), lh, logits, 3, text, pad,
                                  qtts.loop_params(2, stop_on_eos=False), seed=77)
    tok, st = oracle.sample_token(logits, 0.8, 50, 1.05, (0,) * 16, 77)
    assert codes[0, 0] == tok
    sem = ot.embed_codec_token(tok)
    ac = op.generate_acoustic_codes(lh, sem, op.new_kv())
    assert np.array_equal(codes[1:, 0], ac)
    comb = (sem + op.get_acoustic_embeddings_sum(ac)) + text[0]
    out = ot.forward_with_embedding(comb, ot.new_kv(4), 3)
    prev = np.concatenate([[tok], ac]).astype(np.uint32)
    tok2, _ = oracle.sample_token(out[H:], 0.8, 50, 1.05, prev, st)
    assert codes[0, 1] == tok2


@pytest.mark.parametrize("greedy", [True, False])
def test_loop_talker_only_matches_manual_composition(tiny, greedy):
    """The talker-only branch (the legacy feedback, src/generate.rs:225-227):
    each frame samples code 0 with prev_tokens = [previous code 0, 0 x 15],
    then feeds embed_codec_token(code 0) alone to forward_with_embedding at
    the next position; groups 1-15 stay 0.  Composed by hand for 6 frames."""
    tw, pw, ot, op = tiny
    H = TINY_TALKER.hidden
    lh = GOLDEN["talker_step0"][:H].astype(np.float32)
    logits = GOLDEN["talker_step0"][H:].astype(np.float32)
    frames, pos0, seed = 6, 2, 31
    params = qtts.loop_params(frames, greedy=greedy, stop_on_eos=False, talker_only=True)
    kv = ot.new_kv(16)
    codes = oracle.generate_codes(ot, None, kv, None, lh, logits, pos0, None, None, params, seed=seed)
    assert codes.shape == (16, frames) and len(kv) == frames
    assert not codes[1:].any()
    hkv, lg, st, prev = ot.new_kv(16), logits, seed, np.zeros(16, np.uint32)
    for f in range(frames):
        tok, st = oracle.sample_token(lg, 0.8, 50, 1.05, prev, st, greedy=greedy)
        assert codes[0, f] == tok, f
        prev[0] = tok
        lg = ot.forward_with_embedding(ot.embed_codec_token(tok), hkv, pos0 + f)[H:]
    k1, v1 = kv.store()
    k2, v2 = hkv.store()
    assert np.array_equal(k1, k2) and np.array_equal(v1, v2)
