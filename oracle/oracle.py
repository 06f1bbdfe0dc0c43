"""ctypes binding of the CPU oracle (oracle/liboracle.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and
bench.py's CPU-baseline leg, always as the reference the results are
compared with or the timed CPU baseline, never as a product path.  Function names follow the reference's
(src/gemv.rs, src/talker.rs, src/code_predictor.rs, src/generate_new.rs).
"""

from __future__ import annotations

import ctypes as C
import os
import sys
from typing import Optional

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_PKG = os.path.join(os.path.dirname(_HERE), "qora-tts-12hz-1.7b_amd")
if _PKG not in sys.path:
    sys.path.insert(0, _PKG)

import qtts  # noqa: E402  (host weight containers and ctypes views)

# QTTS_ORACLE_LIB names another build of the same sources (the sanitizer
# build of tests/sanitize.mk); the default is the -O3 build of oracle/Makefile.
LIB_PATH = os.environ.get("QTTS_ORACLE_LIB") or os.path.join(_HERE, "liboracle.so")
_lib = None


def _p(a):
    # data_as keeps a reference to the array, so a temporary (a contiguous
    # copy made in the argument list) lives until the foreign call returns
    return None if a is None else a.ctypes.data_as(C.c_void_p)


def load():
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(f"{LIB_PATH} is not built (make -C oracle)")
    lib = C.CDLL(LIB_PATH)
    vp, i32, u32 = C.c_void_p, C.c_int32, C.c_uint32
    Q4P, TVP, PVP = C.POINTER(qtts.Q4View), C.POINTER(qtts.TalkerView), C.POINTER(qtts.PredictorView)
    sig = {
        "qor_available_parallelism": ([], i32),
        "qor_f16_to_f32": ([C.c_uint16], C.c_float),
        "qor_gemv": ([vp, Q4P, vp, i32], None),
        "qor_gemm": ([vp, i32, Q4P, vp, i32], None),
        "qor_embed_lookup": ([Q4P, i32, vp], None),
        "qor_rms_norm_f16": ([vp, vp, i32, vp], None),
        "qor_softmax_raw": ([vp, i32], None),
        "qor_silu": ([C.c_float], C.c_float),
        "qor_qk_norm": ([vp, i32, i32, vp], None),
        "qor_build_rope_table": ([i32, i32, C.c_double, vp, vp], None),
        "qor_rope_split": ([vp, i32, i32, i32, vp, vp], None),
        "qor_kv_new": ([i32, i32, i32, i32], vp),
        "qor_kv_free": ([vp], None),
        "qor_kv_len": ([vp], i32),
        "qor_kv_clear": ([vp], None),
        "qor_kv_load": ([vp, vp, vp, i32], i32),
        "qor_kv_store": ([vp, vp, vp], i32),
        "qor_talker_new": ([TVP], vp),
        "qor_talker_free": ([vp], None),
        "qor_forward_with_embedding": ([vp, vp, vp, i32, vp, i32], i32),
        "qor_prefill_talker_raw": ([vp, vp, i32, vp, vp, i32], i32),
        "qor_apply_codec_head": ([vp, vp, vp, i32], None),
        "qor_embed_codec_token": ([vp, u32, vp], None),
        "qor_predictor_new": ([PVP], vp),
        "qor_predictor_free": ([vp], None),
        "qor_generate_acoustic_codes": ([vp, vp, vp, vp, vp, i32], i32),
        "qor_get_acoustic_embeddings_sum": ([vp, vp, vp], None),
        "qor_simple_rand": ([C.POINTER(C.c_uint64)], C.c_float),
        "qor_decoder_num_samples": ([C.POINTER(qtts.DecoderView), i32], C.c_int64),
        "qor_decode_to_audio": ([C.POINTER(qtts.DecoderView), vp, i32, i32, vp, C.c_int64, C.POINTER(C.c_int64), i32],
                                i32),
        "qor_argmax": ([vp, i32, C.POINTER(u32)], i32),
        "qor_text_new": ([C.POINTER(qtts.TextView)], vp),
        "qor_text_free": ([vp], None),
        "qor_embed_text_token": ([vp, u32, vp, i32], i32),
        "qor_build_custom_voice_prompt": ([vp, vp, i32, vp, i32, u32, u32, vp, vp, C.POINTER(i32), i32], i32),
        "qor_prefill_custom_voice": ([vp, vp, i32, vp, i32, u32, u32, vp, vp, vp, vp, C.POINTER(i32), i32], i32),
        "qor_build_trailing_text": ([vp, vp, i32, vp, C.POINTER(i32), i32], i32),
        "qor_generate_speech_codes": ([vp, vp, vp, i32, vp, i32, u32, u32, vp, vp, vp, C.POINTER(qtts.LoopParams),
                                       C.c_uint64, vp, C.POINTER(i32), i32], i32),
        "qor_dec_causal_conv": ([vp, i32, C.POINTER(qtts.ConvView), vp, i32], None),
        "qor_dec_transposed_conv": ([vp, i32, C.POINTER(qtts.ConvView), vp, i32], i32),
        "qor_dec_depthwise_conv": ([vp, i32, C.POINTER(qtts.ConvView), vp, i32], None),
        "qor_dec_snake": ([vp, i32, i32, vp, vp, vp, i32], None),
        "qor_dec_gelu": ([C.c_float], C.c_float),
        "qor_dec_layer_norm_cf": ([vp, vp, vp, i32, i32, C.c_float, vp], None),
        "qor_dec_rms_norm": ([vp, vp, C.c_float, i32, vp], None),
        "qor_dec_rope": ([vp, i32, i32, i32, vp, vp, i32], None),
        "qor_dec_window_attention": ([vp, vp, vp, i32, i32, i32, i32, vp], None),
        "qor_dec_codebook_lookup": ([C.POINTER(qtts.DecoderView), vp, i32, i32, vp], None),
        "qor_sample_token": ([vp, i32, C.POINTER(qtts.SamplerParams), vp, i32, C.POINTER(C.c_uint64),
                              C.POINTER(u32)], i32),
        "qor_generate_codes": ([vp, vp, vp, vp, vp, vp, i32, vp, i32, vp, C.POINTER(qtts.LoopParams), C.c_uint64,
                                vp, C.POINTER(i32), i32], i32),
        "qor_sample_top_k": ([vp, i32, C.c_float, i32, C.POINTER(C.c_uint64), C.POINTER(u32)], i32),
        "qor_predict_codes": ([vp, vp, vp, vp, i32], i32),
        "qor_forward_talker_decode": ([vp, vp, u32, i32, vp, i32, vp, i32], i32),
        "qor_prefill_talker": ([vp, vp, vp, vp, i32, vp, vp, i32], i32),
    }
    for name, (args, res) in sig.items():
        fn = getattr(lib, name)
        fn.argtypes = args
        fn.restype = res
    _lib = lib
    return lib


class OracleError(RuntimeError):
    def __init__(self, status: int):
        self.status = status
        super().__init__(f"oracle status {qtts.STATUS_NAMES[status]}")


def _check(st: int):
    if st != 0:
        raise OracleError(st)


def f32(a, n=None):
    a = np.ascontiguousarray(a, dtype=np.float32)
    if n is not None:
        assert a.size >= n
    return a


# --- src/gemv.rs ------------------------------------------------------------
def gemv(x, w: "qtts.Q4Weight", nthreads: int = 0) -> np.ndarray:
    x = f32(x, w.k)
    y = np.empty(w.n, dtype=np.float32)
    v = w.view()
    load().qor_gemv(_p(x), C.byref(v), _p(y), nthreads)
    return y


def gemm(x, seq_len: int, w: "qtts.Q4Weight", nthreads: int = 0) -> np.ndarray:
    x = f32(x, seq_len * w.k)
    y = np.empty(seq_len * w.n, dtype=np.float32)
    v = w.view()
    load().qor_gemm(_p(x), seq_len, C.byref(v), _p(y), nthreads)
    return y


def embed_lookup(w: "qtts.Q4Weight", token: int) -> np.ndarray:
    y = np.empty(w.n, dtype=np.float32)
    v = w.view()
    load().qor_embed_lookup(C.byref(v), token, _p(y))
    return y


def rms_norm_f16(x, gamma_f16_bits) -> np.ndarray:
    x = f32(x)
    g = np.ascontiguousarray(gamma_f16_bits, dtype=np.uint16)
    y = np.empty_like(x)
    load().qor_rms_norm_f16(_p(x), _p(g), x.size, _p(y))
    return y


def softmax_raw(s) -> np.ndarray:
    s = f32(s).copy()
    load().qor_softmax_raw(_p(s), s.size)
    return s


def silu(x: float) -> float:
    return float(load().qor_silu(x))


def qk_norm(data, num_heads: int, head_dim: int, gamma_f16_bits) -> np.ndarray:
    d = f32(data).copy()
    g = np.ascontiguousarray(gamma_f16_bits, dtype=np.uint16)
    load().qor_qk_norm(_p(d), num_heads, head_dim, _p(g))
    return d


def build_rope_table(head_dim: int, max_pos: int, theta: float):
    half = head_dim // 2
    c = np.empty(max_pos * half, dtype=np.float32)
    s = np.empty(max_pos * half, dtype=np.float32)
    load().qor_build_rope_table(head_dim, max_pos, theta, _p(c), _p(s))
    return c.reshape(max_pos, half), s.reshape(max_pos, half)


def rope_split(data, num_heads: int, head_dim: int, pos: int, cos_t, sin_t) -> np.ndarray:
    d = f32(data).copy()
    load().qor_rope_split(_p(d), num_heads, head_dim, pos, _p(f32(cos_t)), _p(f32(sin_t)))
    return d


def f16_to_f32(h: int) -> float:
    return float(load().qor_f16_to_f32(h))


def available_parallelism() -> int:
    return int(load().qor_available_parallelism())


# --- src/generate_new.rs ----------------------------------------------------
def simple_rand(state: int):
    st = C.c_uint64(state)
    r = load().qor_simple_rand(C.byref(st))
    return float(r), int(st.value)


def argmax(logits):
    lg = f32(logits)
    out = C.c_uint32(0)
    _check(load().qor_argmax(_p(lg), lg.size, C.byref(out)))
    return int(out.value)


def sample_token(logits, temperature=0.8, top_k=50, repetition_penalty=1.05, prev_tokens=(0,) * 16, rng=0,
                 greedy=False):
    lg = f32(logits)
    prev = np.ascontiguousarray(prev_tokens, dtype=np.uint32)
    p = qtts.SamplerParams(temperature, top_k, repetition_penalty, 1 if greedy else 0)
    st = C.c_uint64(rng)
    tok = C.c_uint32(0)
    _check(load().qor_sample_token(_p(lg), lg.size, C.byref(p), _p(prev), prev.size, C.byref(st), C.byref(tok)))
    return int(tok.value), int(st.value)


def sample_top_k(logits, temperature, top_k, rng=0):
    """sample_top_k of the legacy generator (src/generate.rs:50-84):
    (token, new_rng_state)."""
    lg = f32(logits)
    st = C.c_uint64(rng)
    tok = C.c_uint32(0)
    _check(load().qor_sample_top_k(_p(lg), lg.size, float(temperature), int(top_k), C.byref(st), C.byref(tok)))
    return int(tok.value), int(st.value)


# --- KV, talker, predictor --------------------------------------------------
class Kv:
    def __init__(self, num_layers, num_kv_heads, head_dim, capacity):
        self.shape = (num_layers, num_kv_heads, head_dim)
        self.h = load().qor_kv_new(num_layers, num_kv_heads, head_dim, capacity)

    def __len__(self):
        return int(load().qor_kv_len(self.h))

    def clear(self):
        load().qor_kv_clear(self.h)

    def load(self, k, v, length):
        k, v = f32(k), f32(v)  # keep the contiguous copies alive over the call
        _check(load().qor_kv_load(self.h, _p(k), _p(v), length))

    def store(self):
        L, H, D = self.shape
        n = len(self)
        k = np.empty((L, n, H, D), dtype=np.float32)
        v = np.empty_like(k)
        _check(load().qor_kv_store(self.h, _p(k), _p(v)))
        return k, v

    def __del__(self):
        try:
            load().qor_kv_free(self.h)
        except Exception:
            pass


class Talker:
    def __init__(self, w: "qtts.TalkerWeights", nthreads: int = 0):
        self.w, self.cfg, self.nthreads = w, w.cfg, nthreads
        self._view = w.view()
        self.h = load().qor_talker_new(C.byref(self._view))

    def new_kv(self, capacity):
        c = self.cfg
        return Kv(c.layers, c.kv_heads, c.head_dim, capacity)

    def forward_with_embedding(self, embedding, kv: Kv, position: int) -> np.ndarray:
        e = f32(embedding, self.cfg.hidden)
        out = np.empty(self.cfg.hidden + self.cfg.vocab, dtype=np.float32)
        _check(load().qor_forward_with_embedding(self.h, _p(e), kv.h, position, _p(out), self.nthreads))
        return out

    def prefill_talker_raw(self, x, seq_len: int, kv: Kv) -> np.ndarray:
        x = f32(x, seq_len * self.cfg.hidden)
        out = np.empty(self.cfg.hidden, dtype=np.float32)
        _check(load().qor_prefill_talker_raw(self.h, _p(x), seq_len, kv.h, _p(out), self.nthreads))
        return out

    def apply_codec_head(self, hidden) -> np.ndarray:
        out = np.empty(self.cfg.vocab, dtype=np.float32)
        load().qor_apply_codec_head(self.h, _p(f32(hidden)), _p(out), self.nthreads)
        return out

    def embed_codec_token(self, token: int) -> np.ndarray:
        out = np.empty(self.cfg.hidden, dtype=np.float32)
        load().qor_embed_codec_token(self.h, token, _p(out))
        return out

    def __del__(self):
        try:
            load().qor_talker_free(self.h)
        except Exception:
            pass


class CodePredictor:
    def __init__(self, w: "qtts.CodePredictorWeights", nthreads: int = 0):
        self.w, self.cfg, self.nthreads = w, w.cfg, nthreads
        self.num_groups, self.talker_hidden = w.num_groups, w.talker_hidden
        self._view = w.view()
        self.h = load().qor_predictor_new(C.byref(self._view))

    def new_kv(self, capacity=16):
        c = self.cfg
        return Kv(c.layers, c.kv_heads, c.head_dim, capacity)

    def generate_acoustic_codes(self, talker_hidden, semantic_embed, kv: Kv) -> np.ndarray:
        codes = np.empty(self.num_groups, dtype=np.uint32)
        _check(load().qor_generate_acoustic_codes(self.h, _p(f32(talker_hidden)), _p(f32(semantic_embed)), kv.h,
                                                  _p(codes), self.nthreads))
        return codes

    def get_acoustic_embeddings_sum(self, codes) -> np.ndarray:
        cs = np.ascontiguousarray(codes, dtype=np.uint32)
        out = np.empty(self.talker_hidden, dtype=np.float32)
        load().qor_get_acoustic_embeddings_sum(self.h, _p(cs), _p(out))
        return out

    def predict_codes(self, talker_hidden, kv: Kv) -> np.ndarray:
        """predict_codes (src/code_predictor.rs:126-213): [num_groups][vocab]."""
        out = np.empty((self.num_groups, self.cfg.vocab), dtype=np.float32)
        _check(load().qor_predict_codes(self.h, _p(f32(talker_hidden, self.talker_hidden)), kv.h, _p(out),
                                        self.nthreads))
        return out

    def __del__(self):
        try:
            load().qor_predictor_free(self.h)
        except Exception:
            pass


def generate_codes(talker: Talker, predictor: Optional[CodePredictor], talker_kv: Kv, predictor_kv: Optional[Kv],
                   last_hidden, logits, position: int, trailing_text, tts_pad_embed, params: "qtts.LoopParams",
                   seed: int, nthreads: int = 0) -> np.ndarray:
    hidden = talker.cfg.hidden
    tt = None if trailing_text is None else f32(trailing_text).reshape(-1, hidden)
    tl = 0 if tt is None else tt.shape[0]
    pad = None if tts_pad_embed is None else f32(tts_pad_embed)
    codes = np.zeros((16, max(params.max_codes, 1)), dtype=np.uint32)
    n = C.c_int32(0)
    _check(load().qor_generate_codes(talker.h, predictor.h if predictor is not None else None, talker_kv.h,
                                     predictor_kv.h if predictor_kv is not None else None, _p(f32(last_hidden)), _p(f32(logits)),
                                     position, _p(tt), tl, _p(pad), C.byref(params), seed, _p(codes), C.byref(n),
                                     nthreads))
    return codes[:, : n.value].copy()


# --- prompt assembly (qtts_oracle_prompt.c) ---------------------------------
class Text:
    """The text embedding and projection for a talker (src/talker.rs:33-56)."""

    def __init__(self, talker: Talker, w: "qtts.TextWeights", nthreads: int = 0):
        self.talker, self.w, self.nthreads = talker, w, nthreads
        self._view = w.view()
        self.h = load().qor_text_new(C.byref(self._view))

    @property
    def hidden(self):
        return self.talker.cfg.hidden

    def embed_text_token(self, token: int) -> np.ndarray:
        out = np.empty(self.hidden, dtype=np.float32)
        _check(load().qor_embed_text_token(self.h, token, _p(out), self.nthreads))
        return out

    def _tok(self, tokens):
        t = np.ascontiguousarray(tokens, dtype=np.uint32)
        return t, (_p(t) if t.size else None)

    def build_custom_voice_prompt(self, tokens, speaker_id, language_id, voice=None) -> np.ndarray:
        t, tp = self._tok(tokens)
        rows = np.empty((10, self.hidden), dtype=np.float32)
        n = C.c_int32(0)
        v = None if voice is None else f32(voice)
        _check(load().qor_build_custom_voice_prompt(self.talker.h, self.h, self.talker.cfg.vocab, tp, t.size,
                                                    speaker_id, language_id, _p(v), _p(rows), C.byref(n),
                                                    self.nthreads))
        return rows[: n.value].copy()

    def prefill_custom_voice(self, tokens, speaker_id, language_id, kv: Kv, voice=None):
        t, tp = self._tok(tokens)
        lh = np.empty(self.hidden, dtype=np.float32)
        lg = np.empty(self.talker.cfg.vocab, dtype=np.float32)
        pos = C.c_int32(0)
        v = None if voice is None else f32(voice)
        _check(load().qor_prefill_custom_voice(self.talker.h, self.h, self.talker.cfg.vocab, tp, t.size, speaker_id,
                                               language_id, _p(v), kv.h, _p(lh), _p(lg), C.byref(pos),
                                               self.nthreads))
        return lh, lg, pos.value

    def forward_talker_decode(self, token: int, is_text: bool, kv: Kv, position: int) -> np.ndarray:
        """forward_talker_decode (src/talker.rs:161-258): the final-normed hidden."""
        out = np.empty(self.hidden, dtype=np.float32)
        _check(load().qor_forward_talker_decode(self.talker.h, self.h, token, 1 if is_text else 0, kv.h, position,
                                                _p(out), self.nthreads))
        return out

    def build_trailing_text(self, tokens) -> np.ndarray:
        t, tp = self._tok(tokens)
        rows = np.empty((max(t.size, 1), self.hidden), dtype=np.float32)
        n = C.c_int32(0)
        _check(load().qor_build_trailing_text(self.h, tp, t.size, _p(rows), C.byref(n), self.nthreads))
        return rows[: n.value].copy()

    def generate_speech_codes(self, predictor, tokens, speaker_id, language_id, talker_kv: Kv, predictor_kv,
                              params: "qtts.LoopParams", seed: int, voice=None) -> np.ndarray:
        t, tp = self._tok(tokens)
        codes = np.zeros((16, max(params.max_codes, 1)), dtype=np.uint32)
        n = C.c_int32(0)
        v = None if voice is None else f32(voice)
        _check(load().qor_generate_speech_codes(self.talker.h, predictor.h if predictor is not None else None, self.h,
                                                self.talker.cfg.vocab, tp, t.size, speaker_id, language_id, _p(v),
                                                talker_kv.h, predictor_kv.h if predictor_kv is not None else None,
                                                C.byref(params), seed, _p(codes), C.byref(n), self.nthreads))
        return codes[:, : n.value].copy()

    def __del__(self):
        try:
            load().qor_text_free(self.h)
        except Exception:
            pass


def prefill_talker(talker: Talker, text: Optional[Text], tokens, is_text, kv: Kv, nthreads: int = 0) -> np.ndarray:
    """prefill_talker (src/talker.rs:467-488): the (token, is_text) rows
    embedded by embed_text_token or embed_codec_token, then
    prefill_talker_raw; returns the final-normed last row."""
    t = np.ascontiguousarray(tokens, dtype=np.uint32)
    f = np.ascontiguousarray(np.asarray(is_text, dtype=bool), dtype=np.int32)
    assert t.shape == f.shape
    out = np.empty(talker.cfg.hidden, dtype=np.float32)
    _check(load().qor_prefill_talker(talker.h, text.h if text is not None else None, _p(t) if t.size else None,
                                     _p(f) if f.size else None, t.size, kv.h, _p(out), nthreads))
    return out


def decode_to_audio(w, codes, nthreads: int = 0) -> np.ndarray:
    """decode_to_audio (src/decoder.rs:394-509) of codes [groups][frames] with
    the decoder weights w (anything with .view() -> DecoderView)."""
    codes = np.ascontiguousarray(codes, dtype=np.uint32)
    frames = codes.shape[1]
    view = w.view()
    n_out = int(load().qor_decoder_num_samples(C.byref(view), frames))
    out = np.empty(max(1, n_out), dtype=np.float32)
    n = C.c_int64()
    _check(load().qor_decode_to_audio(C.byref(view), _p(codes), frames, frames, _p(out), out.size, C.byref(n),
                                      nthreads))
    return out[: n.value]


# --- decoder primitives (test hooks of qtts_oracle_decoder.c) ---------------
class dec:
    """The decoder oracle's primitives one by one, for the CPU checks that pin
    them.  Signals are channel-first [C][L] float32 arrays."""

    @staticmethod
    def _cv(weight, bias, cin, cout, k, stride=1, pad=0, dil=1):
        w, b = f32(weight), f32(bias)
        return qtts.ConvView(w.ctypes.data, b.ctypes.data, cin, cout, k, stride, pad, dil), (w, b)

    @staticmethod
    def causal_conv(x, w, b, dilation=1, nthreads=0):
        cout, cin, k = w.shape
        x = f32(x)
        view, keep = dec._cv(w, b, cin, cout, k, 1, 0, dilation)
        out = np.empty((cout, x.shape[1]), dtype=np.float32)
        load().qor_dec_causal_conv(_p(x), x.shape[1], C.byref(view), _p(out), nthreads)
        return out

    @staticmethod
    def transposed_conv(x, w, b, stride, padding=0, nthreads=0):
        cin, cout, k = w.shape
        x = f32(x)
        L = x.shape[1]
        view, keep = dec._cv(w, b, cin, cout, k, stride, padding, 1)
        out = np.empty(cout * ((L - 1) * stride - 2 * padding + k), dtype=np.float32)
        n = load().qor_dec_transposed_conv(_p(x), L, C.byref(view), _p(out), nthreads)
        return out[: cout * n].reshape(cout, n)

    @staticmethod
    def depthwise_conv(x, w, b, padding=0, nthreads=0):
        c, k = w.shape
        x = f32(x)
        view, keep = dec._cv(w, b, c, c, k, 1, padding, 1)
        out = np.empty_like(x)
        load().qor_dec_depthwise_conv(_p(x), x.shape[1], C.byref(view), _p(out), nthreads)
        return out

    @staticmethod
    def snake(x, alpha, beta, nthreads=0):
        x, a, b = f32(x), f32(alpha), f32(beta)
        out = np.empty_like(x)
        load().qor_dec_snake(_p(x), x.shape[0], x.shape[1], _p(a), _p(b), _p(out), nthreads)
        return out

    @staticmethod
    def gelu(x):
        return float(load().qor_dec_gelu(x))

    @staticmethod
    def layer_norm_cf(x, g, b, eps=1e-5):
        x = f32(x)
        out = np.empty_like(x)
        load().qor_dec_layer_norm_cf(_p(x), _p(f32(g)), _p(f32(b)), x.shape[0], x.shape[1], eps, _p(out))
        return out

    @staticmethod
    def rms_norm(x, g, eps=1e-5):
        x = f32(x)
        out = np.empty_like(x)
        load().qor_dec_rms_norm(_p(x), _p(f32(g)), eps, x.size, _p(out))
        return out

    @staticmethod
    def rope(x, heads, hd, pos, cos_t, sin_t):
        d = f32(x).copy()
        c = f32(cos_t)
        load().qor_dec_rope(_p(d), heads, hd, pos, _p(c), _p(f32(sin_t)), c.size // (hd // 2))
        return d

    @staticmethod
    def window_attention(q, k, v, heads, hd, window):
        q, k, v = f32(q), f32(k), f32(v)
        out = np.empty_like(q)
        load().qor_dec_window_attention(_p(q), _p(k), _p(v), q.shape[0], heads, hd, window, _p(out))
        return out

    @staticmethod
    def codebook_lookup(w, codes):
        codes = np.ascontiguousarray(codes, dtype=np.uint32)
        T = codes.shape[1]
        view = w.view()
        out = np.empty((w.cfg.vq_dim, T), dtype=np.float32)
        load().qor_dec_codebook_lookup(C.byref(view), _p(codes), T, T, _p(out))
        return out
