"""Writes tests/golden/golden.npz: known-answer vectors for the per-code path.

The reference holds no test vectors for this path (its only tests are four
mel-filterbank checks in src/audio_features.rs:337-374), so every vector here
comes from a closed form or from the float64 numpy model in
tests/numpy_model.py, never from the oracle or the HIP library:

  f16_*       binary16 rounding of float32 values (numpy's IEEE conversion,
              the `half` 2.7.1 crate's from_f32 semantics)
  xs_*        xorshift64 (13, 7, 17) states and simple_rand values
              (src/generate_new.rs:17-22) from exact integer arithmetic
  rope_*      RoPE table entries cos/sin(pos * theta^(-2i/128)) in float64,
              rounded to float32 (src/rope.rs:11-41)
  gemv_*      a small Q4 GEMV (64 -> 96) from a fixed numpy RNG, float64
  synth_*     a few outputs of the seeded synthetic generator (pins it)
  talker_*    one decode step and a 6-token prefill of the small talker
              (seed 31) from the float64 model
  pred_*      predictor codes and logits of the small predictor (seed 31)

Run from the repository root:  python tests/golden/make_golden.py
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, os.path.join(ROOT, "qora-tts-12hz-1.7b_amd"))
sys.path.insert(0, os.path.dirname(HERE))

import qtts  # noqa: E402  (seeded synthetic weights only)
import numpy_model as nm  # noqa: E402
from shapes import TINY_PREDICTOR, TINY_TALKER  # noqa: E402

MASK = (1 << 64) - 1


def u64_to_f32_rne(x: int) -> np.float32:
    """Round a u64 to the nearest float32 (ties to even), exactly."""
    if x == 0:
        return np.float32(0.0)
    e = x.bit_length() - 24
    if e <= 0:
        return np.float32(x)
    q, r = divmod(x, 1 << e)
    half = 1 << (e - 1)
    if r > half or (r == half and (q & 1)):
        q += 1
    return np.float32(q) * np.float32(2.0) ** e


def xorshift(s: int) -> int:
    s ^= (s << 13) & MASK
    s ^= s >> 7
    s ^= (s << 17) & MASK
    return s


def main():
    out = {}
    rng = np.random.default_rng(20261201)

    # binary16 rounding
    vals = np.concatenate([
        rng.standard_normal(4000).astype(np.float32) * np.float32(0.02),
        (rng.standard_normal(2000) * 1e-5).astype(np.float32),   # subnormal range
        (rng.standard_normal(1000) * 3e4).astype(np.float32),    # near overflow
        np.array([0.0, -0.0, 65504.0, 65519.99, 65520.0, 1e9, 2 ** -24, 2 ** -25, 1.5 * 2 ** -25,
                  2 ** -14, 2 ** -14 - 2 ** -25, 1.0 + 2 ** -11, 1.0 + 3 * 2 ** -11, np.inf, -np.inf],
                 dtype=np.float32),
    ])
    out["f16_in"] = vals.view(np.uint32)
    out["f16_out"] = vals.astype(np.float16).view(np.uint16)

    # xorshift64 / simple_rand
    seeds = [1, 12345, 0x9E3779B97F4A7C15, 0xFFFFFFFFFFFFFFFF, 42, 0x8000000000000000]
    states, rs = [], []
    for s in seeds:
        st, rr = [], []
        for _ in range(8):
            s = xorshift(s)
            st.append(s)
            rr.append(np.float32(u64_to_f32_rne(s) / np.float32(2.0 ** 64)))
        states.append(st)
        rs.append(rr)
    out["xs_seeds"] = np.array(seeds, dtype=np.uint64)
    out["xs_states"] = np.array(states, dtype=np.uint64)
    out["xs_r"] = np.array(rs, dtype=np.float32)

    # RoPE table entries
    pos = np.array([0, 1, 7, 64, 256, 563, 2063, 32767])
    idx = np.array([0, 1, 2, 31, 32, 63])
    ang = pos[:, None].astype(np.float64) * (1.0 / 1.0e6 ** ((2 * idx[None, :]).astype(np.float64) / 128.0))
    out["rope_pos"], out["rope_i"] = pos, idx
    out["rope_cos"], out["rope_sin"] = np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)

    # small Q4 GEMV
    K, N = 64, 96
    packed = rng.integers(0, 256, size=(K, N // 2), dtype=np.uint8)
    scales = np.abs(rng.standard_normal((K, N // 32)) * 0.02).astype(np.float32).astype(np.float16).view(np.uint16)
    x = rng.standard_normal(K).astype(np.float32)
    w = qtts.Q4Weight(packed, scales, K, N)
    out["gemv_packed"], out["gemv_scales"], out["gemv_x"] = packed, scales, x
    out["gemv_y"] = w.dequantize().astype(np.float64).T @ x.astype(np.float64)

    # synthetic generator pins
    out["synth_u64"] = np.array([qtts.load_library().qtts_synth_u64(7, 11, i) for i in range(8)], dtype=np.uint64)
    sw = qtts.Q4Weight.synthetic(3, "golden.synth", 32, 64)
    out["synth_packed"], out["synth_scales"] = sw.packed[:2].copy(), sw.scales[:4].copy()
    out["synth_normal"] = qtts.synth_normal_f32(3, "golden.normal", 16)

    # small talker: one step on an empty cache, then a 6-token prefill
    tw = qtts.TalkerWeights(31, TINY_TALKER)
    tm = nm.TalkerModel(tw)
    emb = qtts.synth_normal_f32(31, "golden.emb", TINY_TALKER.hidden)
    cache = tm.stack.empty_cache()
    step0 = tm.forward_with_embedding(emb, cache, 0)
    emb1 = qtts.synth_normal_f32(31, "golden.emb1", TINY_TALKER.hidden)
    step1 = tm.forward_with_embedding(emb1, cache, 1)
    out["talker_step0"], out["talker_step1"] = step0, step1
    X = qtts.synth_normal_f32(31, "golden.prefill", 6 * TINY_TALKER.hidden).reshape(6, -1)
    out["talker_prefill6"] = tm.prefill(X, tm.stack.empty_cache())

    # small predictor
    pw = qtts.CodePredictorWeights(31, TINY_PREDICTOR, talker_hidden=TINY_TALKER.hidden)
    pm = nm.PredictorModel(pw)
    sem = tw.codec_embedding.dequantize()[11]
    codes, logits = pm.generate_acoustic_codes(step0[: TINY_TALKER.hidden], sem)
    out["pred_codes"], out["pred_logits0"] = codes, logits[0]

    path = os.path.join(HERE, "golden.npz")
    np.savez_compressed(path, **out)
    print(f"wrote {path} ({os.path.getsize(path)} bytes)")


if __name__ == "__main__":
    main()
