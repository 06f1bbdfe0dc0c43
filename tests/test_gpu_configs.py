"""GPU parity at the full 1.7B shapes of the loop workloads, against the
oracle on the same seeded random-init weights and inputs:

- the talker-only loop (the legacy feedback, codec_embedding[code0] as the
  next input, src/generate.rs:225-227): a 64-token prefill, then 64 greedy
  and 64 sampled steps (top-k 50, T 0.8, penalty 1.05); and 64 sampled steps
  from a cache loaded to 500 N(0,1) rows, through position 564;
- the talker + code predictor loop (src/generate_new.rs:242-300) after a
  64-token prefill: 64 greedy and 64 sampled frames;
- two talker steps from caches loaded to 564, 2064 and 8184 N(0,1) rows, on
  the frame engine and on the multi-kernel path (k_attn);
- two talker steps from caches loaded to 16384 and 32766 N(0,1) rows (the
  latter at the last two positions of the 32768-row RoPE table), on both
  paths;
- 16 batched streams (qtts_generate_codes_batch) in 2064-row caches loaded
  to 2000 N(0,1) rows: 3 sampled frames, every stream's codes, frame count,
  cache length and appended cache rows.

Bars: codes identical; hidden states and cache rows within 1e-3 relative
and within the regression bar of tests/shapes.py (about ten times the
measured error).
The oracle loops run in worker threads (ctypes releases the GIL), the
predictor being single-threaded as in the reference.
"""
import time
from concurrent.futures import ThreadPoolExecutor

import numpy as np
import pytest

import qtts
from oracle import oracle
from shapes import FULL_PREDICTOR, FULL_TALKER, rel_err, within

pytestmark = pytest.mark.gpu

REL_TOL = 1e-3
PROMPT = 64


@pytest.fixture(scope="module")
def full(ctx):
    t0 = time.time()
    tw = qtts.TalkerWeights(1, FULL_TALKER)
    pw = qtts.CodePredictorWeights(1, FULL_PREDICTOR, talker_hidden=FULL_TALKER.hidden)
    objs = (tw, pw, qtts.Talker(ctx, tw), qtts.CodePredictor(ctx, pw), oracle.Talker(tw), oracle.CodePredictor(pw))
    print(f"1.7B weights synthesised and uploaded in {time.time() - t0:.1f}s", flush=True)
    return objs


@pytest.fixture(scope="module")
def prompt64(full):
    """A 64-token N(0,1) prompt prefilled on both sides; returns each side's
    cache contents and the oracle's last hidden state and logits (the loop
    inputs both sides start from)."""
    tw, _, t, _, ot, _ = full
    H = tw.cfg.hidden
    x = qtts.synth_normal_f32(40, "cfg3.prompt", PROMPT * H)
    kv, okv = t.new_kv(PROMPT + 8), ot.new_kv(PROMPT + 8)
    lh = t.prefill_talker_raw(x, PROMPT, kv)
    olh = ot.prefill_talker_raw(x, PROMPT, okv)
    print(f"64-token prefill: last hidden rel err {rel_err(lh, olh):.2e}", flush=True)
    assert within(lh, olh)
    gk, gv = kv.store()
    rk, rv = okv.store()
    assert within(gk, rk) and within(gv, rv)
    return {"gpu": (gk, gv), "oracle": (rk, rv), "last_hidden": olh, "logits": ot.apply_codec_head(olh)}


def _caches(t, ot, cap, gpu_kv, oracle_kv, length):
    kv, okv = t.new_kv(cap), ot.new_kv(cap)
    kv.load(gpu_kv[0], gpu_kv[1], length)
    okv.load(oracle_kv[0], oracle_kv[1], length)
    return kv, okv


def _check_appended(kv, okv, start, count):
    """The rows the loop appended to both caches agree."""
    (gk, gv), (rk, rv) = kv.store(), okv.store()
    assert gk.shape == rk.shape
    sl = slice(start, start + count)
    assert within(gk[:, sl], rk[:, sl]) and within(gv[:, sl], rv[:, sl])


@pytest.mark.timeout(600)
@pytest.mark.parametrize("greedy", [True, False], ids=["greedy", "sampled"])
def test_config3_talker_only_after_prefill(full, prompt64, greedy):
    """64 talker-only steps after the 64-token prefill (KV 65 -> 128)."""
    tw, _, t, _, ot, _ = full
    steps = 64
    params = qtts.loop_params(steps, temperature=0.8, top_k=50, repetition_penalty=1.05, greedy=greedy,
                              stop_on_eos=False, talker_only=True)
    kv, okv = _caches(t, ot, PROMPT + steps + 8, prompt64["gpu"], prompt64["oracle"], PROMPT)
    lh, lg = prompt64["last_hidden"], prompt64["logits"]
    t0 = time.time()
    got = qtts.generate_codes(t, None, kv, None, lh, lg, PROMPT, None, None, params, seed=2024)
    ref = oracle.generate_codes(ot, None, okv, None, lh, lg, PROMPT, None, None, params, seed=2024)
    print(f"talker-only {steps} steps ({'greedy' if greedy else 'sampled'}): oracle+gpu {time.time() - t0:.1f}s",
          flush=True)
    assert got.shape == ref.shape == (16, steps)
    assert np.array_equal(got[0], ref[0]), np.argwhere(got[0] != ref[0])[:5]
    assert len(kv) == len(okv) == PROMPT + steps
    _check_appended(kv, okv, PROMPT, steps)


@pytest.mark.timeout(600)
def test_config3_talker_only_to_564(full):
    """64 sampled talker-only steps from a cache loaded to 500 N(0,1) rows:
    the last steps of the 500-step loop, through KV length 564."""
    tw, _, t, _, ot, _ = full
    c = tw.cfg
    L, steps = 500, 64
    shape = (c.layers, L, c.kv_heads, c.head_dim)
    k = qtts.synth_normal_f32(41, "cfg3.k", int(np.prod(shape))).reshape(shape)
    v = qtts.synth_normal_f32(41, "cfg3.v", int(np.prod(shape))).reshape(shape)
    kv, okv = _caches(t, ot, L + steps, (k, v), (k, v), L)
    del k, v
    lh = qtts.synth_normal_f32(41, "cfg3.h", c.hidden)
    lg = ot.apply_codec_head(lh)
    params = qtts.loop_params(steps, temperature=0.8, top_k=50, repetition_penalty=1.05, stop_on_eos=False,
                              talker_only=True)
    got = qtts.generate_codes(t, None, kv, None, lh, lg, L, None, None, params, seed=77)
    ref = oracle.generate_codes(ot, None, okv, None, lh, lg, L, None, None, params, seed=77)
    assert got.shape == ref.shape == (16, steps)
    assert np.array_equal(got[0], ref[0]), np.argwhere(got[0] != ref[0])[:5]
    assert len(kv) == len(okv) == L + steps == 564
    _check_appended(kv, okv, L, steps)


@pytest.mark.timeout(900)
def test_full_loop_64_frames_after_prefill(full, prompt64):
    """The talker + predictor loop, 64 frames after the 64-token prefill,
    greedy and sampled: codes identical for every frame and group."""
    tw, pw, t, p, ot, op = full
    H, frames = tw.cfg.hidden, 64
    lh, lg = prompt64["last_hidden"], prompt64["logits"]
    text = qtts.synth_normal_f32(42, "full.text", 5 * H, 0.0, 0.1).reshape(5, H)
    pad = qtts.synth_normal_f32(42, "full.pad", H, 0.0, 0.1)
    modes = {"greedy": qtts.loop_params(frames, greedy=True, repetition_penalty=1.05, stop_on_eos=False),
             "sampled": qtts.loop_params(frames, temperature=0.8, top_k=50, repetition_penalty=1.05,
                                         stop_on_eos=False)}
    runs = {}
    for name in modes:
        kv, okv = _caches(t, ot, PROMPT + frames + 8, prompt64["gpu"], prompt64["oracle"], PROMPT)
        runs[name] = (kv, okv)

    def oracle_loop(name):
        okv = runs[name][1]
        return oracle.generate_codes(ot, op, okv, op.new_kv(), lh, lg, PROMPT, text, pad, modes[name], seed=555)

    t0 = time.time()
    with ThreadPoolExecutor(max_workers=2) as pool:
        futs = {name: pool.submit(oracle_loop, name) for name in modes}
        got = {name: qtts.generate_codes(t, p, runs[name][0], p.new_kv(), lh, lg, PROMPT, text, pad, modes[name],
                                         seed=555) for name in modes}
        refs = {name: f.result() for name, f in futs.items()}
    print(f"full loop 2 x {frames} frames: {time.time() - t0:.1f}s", flush=True)
    for name in modes:
        assert got[name].shape == refs[name].shape == (16, frames), name
        assert np.array_equal(got[name], refs[name]), (name, np.argwhere(got[name] != refs[name])[:5])
        kv, okv = runs[name]
        assert len(kv) == len(okv) == PROMPT + frames
        _check_appended(kv, okv, PROMPT, frames)


def _loaded_caches(t, ot, c, L, cap, seed, tag):
    """Both sides' caches loaded to the same L N(0,1) rows."""
    shape = (c.layers, L, c.kv_heads, c.head_dim)
    k = qtts.synth_normal_f32(seed, f"{tag}.k", int(np.prod(shape))).reshape(shape)
    v = qtts.synth_normal_f32(seed, f"{tag}.v", int(np.prod(shape))).reshape(shape)
    return _caches(t, ot, cap, (k, v), (k, v), L)


@pytest.mark.timeout(900)
def test_config4_bench_window(full):
    """The window bench.py times: the talker + predictor loop from a cache of
    304 rows (N(0,1)), 20 sampled frames at cache lengths 305..324 (top-k 50,
    T 0.8, penalty 1.05, trailing text then pad): codes identical, appended
    cache rows within the bars."""
    tw, pw, t, p, ot, op = full
    c = tw.cfg
    L, frames = 304, 20
    kv, okv = _loaded_caches(t, ot, c, L, L + frames + 4, 44, "cfg4win")
    lh = qtts.synth_normal_f32(44, "cfg4win.h", c.hidden)
    lg = ot.apply_codec_head(lh)
    text = qtts.synth_normal_f32(44, "cfg4win.text", 4 * c.hidden, 0.0, 0.1).reshape(4, c.hidden)
    pad = qtts.synth_normal_f32(44, "cfg4win.pad", c.hidden, 0.0, 0.1)
    params = qtts.loop_params(frames, temperature=0.8, top_k=50, repetition_penalty=1.05, stop_on_eos=False)
    t0 = time.time()
    with ThreadPoolExecutor(max_workers=1) as pool:
        fut = pool.submit(oracle.generate_codes, ot, op, okv, op.new_kv(), lh, lg, L, text, pad, params, 4242)
        got = qtts.generate_codes(t, p, kv, p.new_kv(), lh, lg, L, text, pad, params, seed=4242)
        ref = fut.result()
    print(f"config 4 at KV {L + 1}..{L + frames}: {time.time() - t0:.1f}s", flush=True)
    assert got.shape == ref.shape == (16, frames)
    assert np.array_equal(got, ref), np.argwhere(got != ref)[:5]
    assert len(kv) == len(okv) == L + frames
    _check_appended(kv, okv, L, frames)


@pytest.mark.timeout(900)
@pytest.mark.parametrize("L,frames,engine", [(8172, 16, "frame"), (20000, 4, "frame"), (20000, 4, "ops")])
def test_loop_long_caches(full, monkeypatch, L, frames, engine):
    """The talker + predictor loop from a cache loaded to L N(0,1) rows:
    8172 rows in an 8192-row cache (the frame engine's talker attention at
    32 splits of up to 256 positions, one launch of 16 codes), and 20000 rows
    (past 32 splits: 79 splits of at most 256 positions, several attention
    tasks per block and a combine step in three rounds), on the frame engine
    and on the multi-kernel path.  Sampled frames: codes identical, appended
    cache rows within the bars."""
    tw, pw, t, p, ot, op = full
    if engine == "ops":
        monkeypatch.setenv("QTTS_ENGINE", "ops")
    c = tw.cfg
    kv, okv = _loaded_caches(t, ot, c, L, L + frames + 4, 46, "past")
    lh = qtts.synth_normal_f32(46, "past.h", c.hidden)
    lg = ot.apply_codec_head(lh)
    text = qtts.synth_normal_f32(46, "past.text", 2 * c.hidden, 0.0, 0.1).reshape(2, c.hidden)
    pad = qtts.synth_normal_f32(46, "past.pad", c.hidden, 0.0, 0.1)
    params = qtts.loop_params(frames, temperature=0.8, top_k=50, repetition_penalty=1.05, stop_on_eos=False)
    t0 = time.time()
    with ThreadPoolExecutor(max_workers=1) as pool:
        fut = pool.submit(oracle.generate_codes, ot, op, okv, op.new_kv(), lh, lg, L, text, pad, params, 4343)
        got = qtts.generate_codes(t, p, kv, p.new_kv(), lh, lg, L, text, pad, params, seed=4343)
        ref = fut.result()
    print(f"loop at KV {L + 1}..{L + frames}: {time.time() - t0:.1f}s", flush=True)
    assert got.shape == ref.shape == (16, frames)
    assert np.array_equal(got, ref), np.argwhere(got != ref)[:5]
    assert len(kv) == len(okv) == L + frames
    _check_appended(kv, okv, L, frames)
    kv.close()


@pytest.mark.timeout(600)
def test_loop_is_deterministic(full):
    """The same loop twice on one context with the same seed and inputs
    (talker + predictor, 24 sampled frames from a 304-row cache): codes, the
    talker's appended cache rows and the predictor cache are identical bit
    for bit."""
    tw, pw, t, p, ot, _ = full
    c = tw.cfg
    L, frames = 304, 24
    lh = qtts.synth_normal_f32(45, "det.h", c.hidden)
    lg = ot.apply_codec_head(lh)
    text = qtts.synth_normal_f32(45, "det.text", 3 * c.hidden, 0.0, 0.1).reshape(3, c.hidden)
    pad = qtts.synth_normal_f32(45, "det.pad", c.hidden, 0.0, 0.1)
    params = qtts.loop_params(frames, temperature=0.8, top_k=50, repetition_penalty=1.05, stop_on_eos=False)
    runs = []
    for _ in range(2):
        kv, _okv = _loaded_caches(t, ot, c, L, L + frames + 4, 45, "det")
        pkv = p.new_kv()
        codes = qtts.generate_codes(t, p, kv, pkv, lh, lg, L, text, pad, params, seed=99)
        k, v = kv.store()
        runs.append((codes, k[:, L:], v[:, L:], pkv.store()))
        kv.close()
    (c0, k0, v0, p0), (c1, k1, v1, p1) = runs
    assert np.array_equal(c0, c1)
    assert np.array_equal(k0, k1) and np.array_equal(v0, v1)
    assert all(np.array_equal(a, b) for a, b in zip(p0, p1))


@pytest.mark.timeout(900)
def test_batch_config5_16_streams_2000_rows(full):
    """16 streams of the talker + predictor in 2064-row caches (the talker
    attention then runs more splits per kv head than at 1000 rows), each
    loaded to 2000 N(0,1) rows of its own, with its own last hidden state,
    trailing text and seed: 3 sampled frames.  Every stream's codes, frame
    count, cache length and appended rows match the oracle's single-stream
    loop."""
    tw, pw, t, p, ot, op = full
    c = tw.cfg
    B, L, cap, frames = 16, 2000, 2064, 3
    H = c.hidden
    shape = (c.layers, L, c.kv_heads, c.head_dim)
    kvs, okvs = [], []
    t0 = time.time()
    for b in range(B):
        k = qtts.synth_normal_f32(43, f"cfg5.k.{b}", int(np.prod(shape))).reshape(shape)
        v = qtts.synth_normal_f32(43, f"cfg5.v.{b}", int(np.prod(shape))).reshape(shape)
        kv, okv = _caches(t, ot, cap, (k, v), (k, v), L)
        kvs.append(kv)
        okvs.append(okv)
        del k, v
    print(f"16 caches of {L} rows loaded in {time.time() - t0:.1f}s", flush=True)
    lh = qtts.synth_normal_f32(43, "cfg5.h", B * H).reshape(B, H)
    lg = np.stack([ot.apply_codec_head(lh[b]) for b in range(B)])
    text = qtts.synth_normal_f32(43, "cfg5.text", B * 2 * H, 0.0, 0.1).reshape(B, 2, H)
    pad = qtts.synth_normal_f32(43, "cfg5.pad", H, 0.0, 0.1)
    seeds = [9000 + 7 * b for b in range(B)]
    params = qtts.loop_params(frames, temperature=0.8, top_k=50, repetition_penalty=1.05, stop_on_eos=False)
    pos = [L] * B

    def oracle_loop(b):
        return oracle.generate_codes(ot, op, okvs[b], op.new_kv(), lh[b], lg[b], L, text[b], pad, params,
                                     seed=seeds[b])

    t0 = time.time()
    with ThreadPoolExecutor(max_workers=8) as pool:
        futs = [pool.submit(oracle_loop, b) for b in range(B)]
        got = qtts.generate_codes_batch(t, p, kvs, lh, lg, pos, text, pad, params, seeds)
        refs = [f.result() for f in futs]
    print(f"batch of {B} x {frames} frames and the oracle's streams: {time.time() - t0:.1f}s", flush=True)
    for b in range(B):
        assert got[b].shape == refs[b].shape == (16, frames), b
        assert np.array_equal(got[b], refs[b]), (b, np.argwhere(got[b] != refs[b])[:5])
        assert len(kvs[b]) == len(okvs[b]) == L + frames, b
        _check_appended(kvs[b], okvs[b], L, frames)


@pytest.mark.timeout(600)
@pytest.mark.parametrize("L", [564, 2064, 8184])
@pytest.mark.parametrize("engine", ["frame", "ops"])
def test_talker_steps_long_cache(full, monkeypatch, L, engine):
    """Two talker steps (forward_with_embedding) from a cache loaded to L
    N(0,1) rows, on the frame engine and on the multi-kernel path (k_attn,
    up to 64 position splits): hidden, logits and the two appended cache rows
    against the oracle.  L = 8184 fills the largest cache the frame engine
    covers with 32 splits (8192 rows: 256 positions each, its score
    buffer's size)."""
    tw, _, t, _, ot, _ = full
    if engine == "ops":
        monkeypatch.setenv("QTTS_ENGINE", "ops")
    c = tw.cfg
    shape = (c.layers, L, c.kv_heads, c.head_dim)
    k = qtts.synth_normal_f32(50 + L, "long.k", int(np.prod(shape))).reshape(shape)
    v = qtts.synth_normal_f32(50 + L, "long.v", int(np.prod(shape))).reshape(shape)
    kv, okv = t.new_kv(L + 8), ot.new_kv(L + 8)
    kv.load(k, v, L)
    okv.load(k, v, L)
    del k, v
    for i in range(2):
        emb = qtts.synth_normal_f32(60 + i, "long.emb", c.hidden)
        got = t.forward_with_embedding(emb, kv, L + i)
        ref = ot.forward_with_embedding(emb, okv, L + i)
        print(f"L={L} {engine} step {i}: hidden rel err {rel_err(got[: c.hidden], ref[: c.hidden]):.2e}", flush=True)
        # measured up to 2.3e-5 at 2064 random rows (long softmax sums)
        tight = 1e-4 if L > 1024 else None
        assert within(got[: c.hidden], ref[: c.hidden], tight) and within(got[c.hidden:], ref[c.hidden:], tight)
    gk, gv = kv.store()
    rk, rv = okv.store()
    assert within(gk[:, L:], rk[:, L:], tight) and within(gv[:, L:], rv[:, L:], tight)
    kv.close()


# The appended rows of the later layers carry the error of softmax sums over
# 16K-32K random positions taken in another order (measured up to 6.3e-5 on
# the multi-kernel path and 4.4e-5 on the frame engine at 16384 rows, against
# ~1e-6 in the hidden state).
CACHE_ROWS_TIGHT = 5e-4


@pytest.mark.timeout(900)
@pytest.mark.parametrize("L", [16384, 32766])
@pytest.mark.parametrize("engine", ["frame", "ops"])
def test_talker_steps_max_context(full, monkeypatch, L, engine):
    """Caches past 16384 rows, up to the maximum: two talker steps at
    positions L and L + 1 -- at L = 32766 the last rows of the 32768-row
    RoPE table (src/rope.rs:11-41) -- from a cache loaded to L N(0,1) rows
    in an (L + 2)-row capacity (7.5 GB of K/V at the maximum).  Both paths
    keep every attention split within 256 positions, their score buffers'
    size: the frame engine with 65 and 128 splits (4 attention tasks per
    block, the combine in rounds of 32 splits), the multi-kernel path's
    one-row k_attn with 65 and 128 splits.  Hidden, logits and the two
    appended cache rows against the oracle."""
    tw, _, t, _, ot, _ = full
    if engine == "ops":
        monkeypatch.setenv("QTTS_ENGINE", "ops")
    c = tw.cfg
    cap = L + 2
    assert cap <= c.max_position
    shape = (c.layers, L, c.kv_heads, c.head_dim)
    t0 = time.time()
    kv, okv = t.new_kv(cap), ot.new_kv(cap)
    k = qtts.synth_normal_f32(71 + L, "max.k", int(np.prod(shape))).reshape(shape)
    v = qtts.synth_normal_f32(71 + L, "max.v", int(np.prod(shape))).reshape(shape)
    kv.load(k, v, L)
    okv.load(k, v, L)
    del k, v
    print(f"caches loaded in {time.time() - t0:.1f}s", flush=True)
    for i in range(2):
        emb = qtts.synth_normal_f32(72 + i, "max.emb", c.hidden)
        got = t.forward_with_embedding(emb, kv, L + i)
        ref = ot.forward_with_embedding(emb, okv, L + i)
        eh, el = rel_err(got[: c.hidden], ref[: c.hidden]), rel_err(got[c.hidden:], ref[c.hidden:])
        print(f"position {L + i}: hidden rel err {eh:.2e}, logits {el:.2e}", flush=True)
        # measured <= 1.3e-6 (1.7e-3 while the 64-split cap let a split
        # overrun the score buffer)
        assert within(got[: c.hidden], ref[: c.hidden]) and within(got[c.hidden:], ref[c.hidden:])
    assert len(kv) == len(okv) == cap
    gk, gv = kv.store()
    rk, rv = okv.store()
    ek, ev = rel_err(gk[:, L:], rk[:, L:]), rel_err(gv[:, L:], rv[:, L:])
    print(f"appended rows: k rel err {ek:.2e}, v {ev:.2e}", flush=True)
    assert within(gk[:, L:], rk[:, L:], CACHE_ROWS_TIGHT) and within(gv[:, L:], rv[:, L:], CACHE_ROWS_TIGHT)
    kv.close()
