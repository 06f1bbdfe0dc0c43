"""Python mirror of the reference crate's per-code-loop API over the C-ABI.

The reference (qora-tts 0.1.0, Rust) exposes its hot path as plain functions:
``gemv``/``gemm`` (src/gemv.rs:148-162), ``forward_with_embedding``
(src/talker.rs:263), ``prefill_talker_raw`` (src/talker.rs:364),
``generate_acoustic_codes`` (src/code_predictor.rs:218), ``sample_token`` and
the frame loop of ``generate_speech`` (src/generate_new.rs:191-391).  This
module exposes the same names over ``lib/libqtts.so`` (include/qtts.h), plus
the host-side weight containers in the reference layout and the seeded
synthetic checkpoints used by the benchmark and tests.

Everything here runs the HIP library; there is no CPU fallback.  Loading
raises if the shared library has not been built.
"""

from __future__ import annotations

import ctypes as C
import dataclasses
import os
import weakref
from typing import List, Optional, Sequence

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "lib", "libqtts.so")

QTTS_OK, QTTS_EINVAL, QTTS_ESHAPE, QTTS_ENOMEM, QTTS_EDEVICE, QTTS_ENAN, QTTS_ERANGE, QTTS_ESTATE = range(8)
STATUS_NAMES = ["OK", "EINVAL", "ESHAPE", "ENOMEM", "EDEVICE", "ENAN", "ERANGE", "ESTATE"]

# Special codec tokens, src/generate_new.rs:34-36.
CODEC_PAD, CODEC_BOS, CODEC_EOS = 2148, 2149, 2150


class QttsError(RuntimeError):
    def __init__(self, status: int, message: str):
        self.status = status
        name = STATUS_NAMES[status] if 0 <= status < len(STATUS_NAMES) else str(status)
        super().__init__(f"qtts {name}: {message}")


class _DeviceObject:
    """A handle owned by a Context: close() frees it once (the context's
    close() calls it for every object still open)."""

    _free_fn = ""

    def _register(self, ctx: "Context", h):
        self.ctx, self.h = ctx, h
        ctx._children.add(self)

    def close(self):
        h = getattr(self, "h", None)
        if h:
            self.h = None
            getattr(self.ctx.lib, self._free_fn)(h)

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


# ---------------------------------------------------------------------------
# ctypes mirror of include/qtts.h
# ---------------------------------------------------------------------------
class Q4View(C.Structure):
    _fields_ = [("packed", C.c_void_p), ("scales", C.c_void_p), ("k", C.c_int32), ("n", C.c_int32)]


class LayerView(C.Structure):
    _fields_ = [(n, Q4View) for n in ("q_proj", "k_proj", "v_proj", "o_proj", "gate_proj", "up_proj", "down_proj")] + [
        (n, C.c_void_p) for n in ("q_norm", "k_norm", "input_norm_gamma", "post_attn_norm_gamma")
    ]


class TalkerView(C.Structure):
    _fields_ = [
        ("num_layers", C.c_int32),
        ("layers", C.POINTER(LayerView)),
        ("codec_embedding", Q4View),
        ("codec_head", Q4View),
        ("final_norm_gamma", C.c_void_p),
        ("hidden_size", C.c_int32),
        ("num_heads", C.c_int32),
        ("num_kv_heads", C.c_int32),
        ("head_dim", C.c_int32),
        ("rope_theta", C.c_double),
        ("max_position", C.c_int32),
        ("rope_cos", C.c_void_p),
        ("rope_sin", C.c_void_p),
    ]


class PredictorView(C.Structure):
    _fields_ = [
        ("input_proj", Q4View),
        ("input_proj_bias", C.c_void_p),
        ("num_groups", C.c_int32),
        ("codec_embeddings", C.POINTER(Q4View)),
        ("num_layers", C.c_int32),
        ("layers", C.POINTER(LayerView)),
        ("lm_heads", C.POINTER(Q4View)),
        ("final_norm_gamma", C.c_void_p),
        ("hidden_size", C.c_int32),
        ("num_heads", C.c_int32),
        ("num_kv_heads", C.c_int32),
        ("head_dim", C.c_int32),
        ("rope_theta", C.c_double),
        ("max_position", C.c_int32),
        ("rope_cos", C.c_void_p),
        ("rope_sin", C.c_void_p),
    ]


class ConvView(C.Structure):
    _fields_ = [("weight", C.c_void_p), ("bias", C.c_void_p)] + [
        (n, C.c_int32) for n in ("in_channels", "out_channels", "kernel_size", "stride", "padding", "dilation")]


class DecLayerView(C.Structure):
    _fields_ = [(n, C.c_void_p) for n in ("q_proj", "k_proj", "v_proj", "o_proj", "gate_proj", "up_proj",
                                          "down_proj", "input_norm", "post_attn_norm", "attn_scale", "mlp_scale")]


class UpsampleView(C.Structure):
    _fields_ = [("channels", C.c_int32), ("inner_dim", C.c_int32), ("conv_t", ConvView), ("dw_conv", ConvView)] + [
        (n, C.c_void_p) for n in ("norm_w", "norm_b", "pw1_w", "pw1_b", "pw2_w", "pw2_b", "gamma")]


class VocosResidualView(C.Structure):
    _fields_ = [("act1_alpha", C.c_void_p), ("act1_beta", C.c_void_p), ("conv1", ConvView),
                ("act2_alpha", C.c_void_p), ("act2_beta", C.c_void_p), ("conv2", ConvView)]


class VocosBlockView(C.Structure):
    _fields_ = [("pre_snake_alpha", C.c_void_p), ("pre_snake_beta", C.c_void_p), ("upsample", ConvView),
                ("num_residuals", C.c_int32), ("residuals", C.POINTER(VocosResidualView))]


class DecoderView(C.Structure):
    _fields_ = [(n, C.c_int32) for n in ("hidden_size", "num_heads", "head_dim", "intermediate_size",
                                         "sliding_window", "codebook_dim", "codebook_size", "vq_dim")] + [
        ("first_codebook", C.c_void_p), ("first_output_proj", C.c_void_p), ("num_rest", C.c_int32),
        ("rest_codebooks", C.POINTER(C.c_void_p)), ("rest_output_proj", C.c_void_p), ("pre_conv", ConvView),
        ("tf_input_w", C.c_void_p), ("tf_input_b", C.c_void_p), ("num_layers", C.c_int32),
        ("layers", C.POINTER(DecLayerView)), ("tf_norm", C.c_void_p), ("tf_output_w", C.c_void_p),
        ("tf_output_b", C.c_void_p), ("num_upsample", C.c_int32), ("upsample", C.POINTER(UpsampleView)),
        ("vocos_init", ConvView), ("num_vocos_blocks", C.c_int32), ("vocos_blocks", C.POINTER(VocosBlockView)),
        ("final_snake_alpha", C.c_void_p), ("final_snake_beta", C.c_void_p), ("output_conv", ConvView),
        ("rope_cos", C.c_void_p), ("rope_sin", C.c_void_p), ("rope_rows", C.c_int32),
    ]


class TextView(C.Structure):
    _fields_ = [
        ("text_embedding", Q4View),
        ("text_proj_fc1", Q4View),
        ("text_proj_fc1_bias", C.c_void_p),
        ("text_proj_fc2", Q4View),
        ("text_proj_fc2_bias", C.c_void_p),
        ("text_hidden_size", C.c_int32),
    ]


class FileInfo(C.Structure):
    _fields_ = [
        ("version", C.c_uint32),
        ("format_id", C.c_uint32),
        ("talker_num_kv_groups", C.c_int32),
        ("predictor_num_kv_groups", C.c_int32),
        ("mrope_sections", C.c_int32),
        ("mrope_section", C.c_int32 * 8),
        ("predictor_has_input_proj", C.c_int32),
    ] + [(n, C.c_int32) for n in (
        "decoder_hidden_size", "decoder_num_heads", "decoder_head_dim", "decoder_intermediate_size",
        "decoder_sliding_window", "decoder_codebook_dim", "decoder_rest_codebooks", "decoder_layers",
        "decoder_upsample_stages", "decoder_vocos_blocks")] + [(n, C.c_int64) for n in (
        "talker_offset", "predictor_offset", "decoder_offset", "decoder_end", "file_bytes", "trailing_bytes")]


class SamplerParams(C.Structure):
    _fields_ = [
        ("temperature", C.c_float),
        ("top_k", C.c_int32),
        ("repetition_penalty", C.c_float),
        ("greedy", C.c_int32),
    ]


class LoopParams(C.Structure):
    _fields_ = [
        ("max_codes", C.c_int32),
        ("sampler", SamplerParams),
        ("codec_eos_id", C.c_uint32),
        ("stop_on_eos", C.c_int32),
        ("talker_only", C.c_int32),
    ]


_lib = None


def _ptr(a: Optional[np.ndarray]):
    # data_as keeps a reference to the array, so a temporary (a contiguous
    # copy made in the argument list) lives until the foreign call returns
    return None if a is None else a.ctypes.data_as(C.c_void_p)


def load_library(path: str = LIB_PATH):
    """Loads libqtts.so; raises if it is missing (no fallback path exists)."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(path):
        raise RuntimeError(f"{path} is not built; run __graft_entry__.build() first")
    lib = C.CDLL(path)
    vp, i32, u32, u64, f32p = C.c_void_p, C.c_int32, C.c_uint32, C.c_uint64, C.c_void_p
    sig = {
        "qtts_version": ([], C.c_char_p),
        "qtts_ctx_create": ([i32, C.POINTER(vp)], i32),
        "qtts_ctx_destroy": ([vp], None),
        "qtts_last_error": ([vp], C.c_char_p),
        "qtts_ctx_stream": ([vp], vp),
        "qtts_ctx_synchronize": ([vp], i32),
        "qtts_q4_upload": ([vp, C.POINTER(Q4View), C.POINTER(vp)], i32),
        "qtts_q4_free": ([vp], None),
        "qtts_q4_bytes": ([vp], C.c_size_t),
        "qtts_gemv": ([vp, vp, f32p, f32p], i32),
        "qtts_gemm": ([vp, vp, f32p, i32, f32p], i32),
        "qtts_embed_lookup": ([vp, vp, i32, f32p], i32),
        "qtts_gemv_device": ([vp, vp, vp, vp], i32),
        "qtts_gemm_device": ([vp, vp, vp, i32, vp], i32),
        "qtts_gemv_device_static": ([vp, vp, i32, vp, vp], i32),
        "qtts_talker_text_upload": ([vp, C.POINTER(TextView)], i32),
        "qtts_embed_text_token": ([vp, u32, vp], i32),
        "qtts_build_custom_voice_prompt": ([vp, vp, i32, u32, u32, vp, vp, C.POINTER(i32)], i32),
        "qtts_prefill_custom_voice": ([vp, vp, i32, u32, u32, vp, vp, vp, vp, C.POINTER(i32)], i32),
        "qtts_build_trailing_text": ([vp, vp, i32, vp, C.POINTER(i32)], i32),
        "qtts_generate_speech_codes": ([vp, vp, vp, i32, u32, u32, vp, vp, vp, C.POINTER(LoopParams), C.c_uint64,
                                        vp, C.POINTER(i32)], i32),
        "qtts_kv_create": ([vp, i32, i32, i32, i32, C.POINTER(vp)], i32),
        "qtts_kv_free": ([vp], None),
        "qtts_kv_len": ([vp], i32),
        "qtts_kv_clear": ([vp], i32),
        "qtts_kv_load": ([vp, f32p, f32p, i32], i32),
        "qtts_kv_store": ([vp, f32p, f32p], i32),
        "qtts_talker_upload": ([vp, C.POINTER(TalkerView), C.POINTER(vp)], i32),
        "qtts_talker_free": ([vp], None),
        "qtts_forward_with_embedding": ([vp, f32p, vp, i32, f32p], i32),
        "qtts_prefill_talker_raw": ([vp, f32p, i32, vp, f32p], i32),
        "qtts_apply_codec_head": ([vp, f32p, f32p], i32),
        "qtts_embed_codec_token": ([vp, u32, f32p], i32),
        "qtts_predictor_upload": ([vp, C.POINTER(PredictorView), C.POINTER(vp)], i32),
        "qtts_predictor_free": ([vp], None),
        "qtts_generate_acoustic_codes": ([vp, f32p, f32p, vp, vp], i32),
        "qtts_get_acoustic_embeddings_sum": ([vp, vp, f32p], i32),
        "qtts_sample_token": ([vp, f32p, i32, C.POINTER(SamplerParams), vp, i32, C.POINTER(u64), C.POINTER(u32)], i32),
        "qtts_sample_top_k": ([vp, f32p, i32, C.c_float, i32, C.POINTER(u64), C.POINTER(u32)], i32),
        "qtts_predict_codes": ([vp, f32p, vp, f32p], i32),
        "qtts_forward_talker_decode": ([vp, u32, i32, vp, i32, f32p], i32),
        "qtts_generate_codes": (
            [vp, vp, vp, vp, f32p, f32p, i32, f32p, i32, f32p, C.POINTER(LoopParams), u64, vp, C.POINTER(i32)],
            i32,
        ),
        "qtts_synth_u64": ([u64, u64, u64], u64),
        "qtts_synth_q4": ([u64, u64, i32, i32, C.c_float, vp, vp], None),
        "qtts_synth_normal_f32": ([u64, u64, C.c_int64, C.c_float, C.c_float, vp], None),
        "qtts_synth_normal_f16": ([u64, u64, C.c_int64, C.c_float, C.c_float, vp], None),
        "qtts_f32_to_f16": ([C.c_float], C.c_uint16),
        "qtts_f16_to_f32": ([C.c_uint16], C.c_float),
        "qtts_stream_read_device": ([vp, u64, vp], i32),
        "qtts_stream_read_device_ex": ([vp, u64, i32, i32, vp], i32),
        "qtts_quantize_f32_to_q4": ([vp, i32, i32, vp, vp], None),
        "qtts_generate_codes_batch": (
            [vp, vp, i32, C.POINTER(vp), f32p, f32p, vp, f32p, i32, f32p, C.POINTER(LoopParams), vp, vp, vp], i32),
        "qtts_model_file_open": ([C.c_char_p, C.POINTER(vp)], i32),
        "qtts_model_file_error": ([], C.c_char_p),
        "qtts_model_file_close": ([vp], None),
        "qtts_model_file_talker": ([vp], C.POINTER(TalkerView)),
        "qtts_model_file_predictor": ([vp], C.POINTER(PredictorView)),
        "qtts_model_file_text": ([vp], C.POINTER(TextView)),
        "qtts_model_file_info": ([vp], C.POINTER(FileInfo)),
        "qtts_model_file_decoder": ([vp], C.POINTER(DecoderView)),
        "qtts_decoder_upload": ([vp, C.POINTER(DecoderView), C.POINTER(vp)], i32),
        "qtts_decoder_free": ([vp], None),
        "qtts_decoder_num_samples": ([vp, i32], C.c_int64),
        "qtts_decode_to_audio": ([vp, vp, i32, i32, f32p, C.c_int64, C.POINTER(C.c_int64)], i32),
        "qtts_decode_to_audio_device": ([vp, vp, i32, i32, vp, C.c_int64, C.POINTER(C.c_int64)], i32),
        "qtts_prefill_talker": ([vp, vp, vp, i32, vp, f32p], i32),
        "qtts_generate_speech": ([vp, vp, vp, vp, i32, u32, u32, vp, vp, vp, C.POINTER(LoopParams), C.c_uint64, f32p,
                                  C.c_int64, C.POINTER(C.c_int64), C.POINTER(i32)], i32),
    }
    for name, (args, res) in sig.items():
        fn = getattr(lib, name)
        fn.argtypes = args
        fn.restype = res
    _lib = lib
    return lib


def exported_symbols() -> List[str]:
    """Names the C-ABI headers declare (checked against the library)."""
    return [
        "qtts_version", "qtts_ctx_create", "qtts_ctx_destroy", "qtts_last_error", "qtts_ctx_stream",
        "qtts_ctx_synchronize", "qtts_q4_upload", "qtts_q4_free", "qtts_q4_bytes", "qtts_gemv", "qtts_gemm",
        "qtts_embed_lookup", "qtts_gemv_device", "qtts_gemm_device", "qtts_gemv_device_static",
        "qtts_talker_text_upload", "qtts_embed_text_token", "qtts_build_custom_voice_prompt", "qtts_prefill_custom_voice",
        "qtts_build_trailing_text", "qtts_generate_speech_codes", "qtts_kv_create", "qtts_kv_free",
        "qtts_kv_len", "qtts_kv_clear", "qtts_kv_load", "qtts_kv_store", "qtts_talker_upload", "qtts_talker_free",
        "qtts_forward_with_embedding", "qtts_prefill_talker_raw", "qtts_apply_codec_head",
        "qtts_embed_codec_token", "qtts_predictor_upload", "qtts_predictor_free", "qtts_generate_acoustic_codes",
        "qtts_get_acoustic_embeddings_sum", "qtts_sample_token", "qtts_sample_top_k", "qtts_predict_codes",
        "qtts_forward_talker_decode", "qtts_generate_codes", "qtts_synth_u64",
        "qtts_synth_q4", "qtts_synth_normal_f32", "qtts_synth_normal_f16", "qtts_f32_to_f16", "qtts_f16_to_f32",
        "qtts_stream_read_device", "qtts_stream_read_device_ex",
        "qtts_quantize_f32_to_q4", "qtts_generate_codes_batch", "qtts_model_file_open", "qtts_model_file_error", "qtts_model_file_close",
        "qtts_model_file_talker", "qtts_model_file_predictor", "qtts_model_file_text", "qtts_model_file_info",
        "qtts_model_file_decoder", "qtts_decoder_upload", "qtts_decoder_free", "qtts_decoder_num_samples",
        "qtts_decode_to_audio", "qtts_decode_to_audio_device", "qtts_prefill_talker", "qtts_generate_speech",
    ]


# ---------------------------------------------------------------------------
# Host weights in the reference layout
# ---------------------------------------------------------------------------
def stream_id(name: str) -> int:
    """Stable 64-bit id of a tensor name (FNV-1a) for the synthetic generator."""
    h = 0xCBF29CE484222325
    for b in name.encode():
        h = ((h ^ b) * 0x100000001B3) & 0xFFFFFFFFFFFFFFFF
    return h


def synth_normal_f32(seed: int, name: str, count: int, mean: float = 0.0, std: float = 1.0) -> np.ndarray:
    out = np.empty(count, dtype=np.float32)
    load_library().qtts_synth_normal_f32(seed, stream_id(name), count, mean, std, _ptr(out))
    return out


def synth_normal_f16(seed: int, name: str, count: int, mean: float = 1.0, std: float = 0.1) -> np.ndarray:
    out = np.empty(count, dtype=np.uint16)
    load_library().qtts_synth_normal_f16(seed, stream_id(name), count, mean, std, _ptr(out))
    return out


class Q4Weight:
    """Q4Weight (src/gemv.rs:26-31): packed [k][n/2] u8, scales [k][n/32] f16 bits."""

    def __init__(self, packed: np.ndarray, scales: np.ndarray, k: int, n: int):
        assert n % 32 == 0
        self.packed = np.ascontiguousarray(packed, dtype=np.uint8).reshape(k, n // 2)
        self.scales = np.ascontiguousarray(scales, dtype=np.uint16).reshape(k, n // 32)
        self.k, self.n = k, n

    @staticmethod
    def synthetic(seed: int, name: str, k: int, n: int, scale_std: float = 0.02) -> "Q4Weight":
        packed = np.empty((k, n // 2), dtype=np.uint8)
        scales = np.empty((k, n // 32), dtype=np.uint16)
        load_library().qtts_synth_q4(seed, stream_id(name), k, n, scale_std, _ptr(packed), _ptr(scales))
        return Q4Weight(packed, scales, k, n)

    @staticmethod
    def quantize(data: np.ndarray) -> "Q4Weight":
        """quantize_f32_to_q4 (src/gemv.rs:92-130)."""
        data = np.ascontiguousarray(data, dtype=np.float32)
        k, n = data.shape
        packed = np.empty((k, n // 2), dtype=np.uint8)
        scales = np.empty((k, n // 32), dtype=np.uint16)
        load_library().qtts_quantize_f32_to_q4(_ptr(data), k, n, _ptr(packed), _ptr(scales))
        return Q4Weight(packed, scales, k, n)

    def nibbles(self) -> np.ndarray:
        lo = self.packed & 0x0F
        hi = self.packed >> 4
        return np.stack([lo, hi], axis=-1).reshape(self.k, self.n)

    def dequantize(self) -> np.ndarray:
        """(nib - 8) * f32(scale), exactly as embed_lookup_q4 (src/gemv.rs:377-400)."""
        s = self.scales.view(np.float16).astype(np.float32)
        s = np.repeat(s, 32, axis=1)
        return (self.nibbles().astype(np.int32) - 8).astype(np.float32) * s

    def view(self) -> Q4View:
        return Q4View(self.packed.ctypes.data, self.scales.ctypes.data, self.k, self.n)

    @property
    def memory_bytes(self) -> int:
        return self.packed.size + 2 * self.scales.size


@dataclasses.dataclass
class StackConfig:
    layers: int
    hidden: int
    heads: int
    kv_heads: int
    head_dim: int
    inter: int
    vocab: int
    max_position: int
    rope_theta: float = 1.0e6


# The 1.7B shapes (src/config.rs:130-153, model/1.7B/config.json).
TALKER_1P7B = StackConfig(layers=28, hidden=2048, heads=16, kv_heads=8, head_dim=128, inter=6144, vocab=3072,
                          max_position=32768)
PREDICTOR_1P7B = StackConfig(layers=5, hidden=1024, heads=16, kv_heads=8, head_dim=128, inter=3072, vocab=2048,
                             max_position=65536)
NUM_GROUPS = 15


class LayerWeights:
    """TalkerLayerWeights / PredictorLayerWeights (src/talker.rs:19-31)."""

    def __init__(self, seed: int, prefix: str, cfg: StackConfig, scale_std: float = 0.02):
        qd, kd = cfg.heads * cfg.head_dim, cfg.kv_heads * cfg.head_dim
        w = lambda n, k, nn: Q4Weight.synthetic(seed, f"{prefix}.{n}", k, nn, scale_std)
        self.q_proj = w("q_proj", cfg.hidden, qd)
        self.k_proj = w("k_proj", cfg.hidden, kd)
        self.v_proj = w("v_proj", cfg.hidden, kd)
        self.o_proj = w("o_proj", qd, cfg.hidden)
        self.gate_proj = w("gate_proj", cfg.hidden, cfg.inter)
        self.up_proj = w("up_proj", cfg.hidden, cfg.inter)
        self.down_proj = w("down_proj", cfg.inter, cfg.hidden)
        self.q_norm = synth_normal_f16(seed, f"{prefix}.q_norm", cfg.head_dim)
        self.k_norm = synth_normal_f16(seed, f"{prefix}.k_norm", cfg.head_dim)
        self.input_norm_gamma = synth_normal_f16(seed, f"{prefix}.input_norm", cfg.hidden)
        self.post_attn_norm_gamma = synth_normal_f16(seed, f"{prefix}.post_attn_norm", cfg.hidden)

    def view(self) -> LayerView:
        v = LayerView()
        for n in ("q_proj", "k_proj", "v_proj", "o_proj", "gate_proj", "up_proj", "down_proj"):
            setattr(v, n, getattr(self, n).view())
        for n in ("q_norm", "k_norm", "input_norm_gamma", "post_attn_norm_gamma"):
            setattr(v, n, getattr(self, n).ctypes.data)
        return v

    @property
    def memory_bytes(self) -> int:
        q4 = sum(getattr(self, n).memory_bytes for n in ("q_proj", "k_proj", "v_proj", "o_proj", "gate_proj",
                                                         "up_proj", "down_proj"))
        return q4 + 2 * (self.q_norm.size + self.k_norm.size + self.input_norm_gamma.size +
                         self.post_attn_norm_gamma.size)


class TalkerWeights:
    """Decode-path part of TalkerWeights (src/talker.rs:33-56), random init."""

    def __init__(self, seed: int, cfg: StackConfig = TALKER_1P7B, scale_std: float = 0.02):
        self.cfg = cfg
        self.layers = [LayerWeights(seed, f"talker.layers.{i}", cfg, scale_std) for i in range(cfg.layers)]
        self.codec_embedding = Q4Weight.synthetic(seed, "talker.codec_embedding", cfg.vocab, cfg.hidden, scale_std)
        self.codec_head = Q4Weight.synthetic(seed, "talker.codec_head", cfg.hidden, cfg.vocab, scale_std)
        self.final_norm_gamma = synth_normal_f16(seed, "talker.final_norm", cfg.hidden)
        self._keep = None

    def view(self) -> TalkerView:
        # Built once: the oracle keeps pointers into these ctypes arrays.
        if self._keep is None:
            arr = (LayerView * len(self.layers))(*[l.view() for l in self.layers])
            c = self.cfg
            v = TalkerView(len(self.layers), arr, self.codec_embedding.view(), self.codec_head.view(),
                           self.final_norm_gamma.ctypes.data, c.hidden, c.heads, c.kv_heads, c.head_dim,
                           c.rope_theta, c.max_position)
            self._keep = (arr, v)
        return self._keep[1]

    @property
    def memory_bytes(self) -> int:
        return (sum(l.memory_bytes for l in self.layers) + self.codec_embedding.memory_bytes +
                self.codec_head.memory_bytes + 2 * self.final_norm_gamma.size)


class CodePredictorWeights:
    """CodePredictorWeights (src/code_predictor.rs:28-46), random init."""

    def __init__(self, seed: int, cfg: StackConfig = PREDICTOR_1P7B, talker_hidden: int = 2048,
                 num_groups: int = NUM_GROUPS, scale_std: float = 0.02):
        self.cfg = cfg
        self.num_groups = num_groups
        self.talker_hidden = talker_hidden
        self.input_proj = Q4Weight.synthetic(seed, "cp.input_proj", talker_hidden, cfg.hidden, scale_std)
        self.input_proj_bias = synth_normal_f32(seed, "cp.input_proj_bias", cfg.hidden, 0.0, 0.02)
        self.codec_embeddings = [Q4Weight.synthetic(seed, f"cp.codec_embedding.{g}", cfg.vocab, talker_hidden,
                                                    scale_std) for g in range(num_groups)]
        self.layers = [LayerWeights(seed, f"cp.layers.{i}", cfg, scale_std) for i in range(cfg.layers)]
        self.lm_heads = [Q4Weight.synthetic(seed, f"cp.lm_head.{g}", cfg.hidden, cfg.vocab, scale_std)
                         for g in range(num_groups)]
        self.final_norm_gamma = synth_normal_f16(seed, "cp.final_norm", cfg.hidden)
        self._keep = None

    def view(self) -> PredictorView:
        # Built once: the oracle keeps pointers into these ctypes arrays.
        if self._keep is None:
            layers = (LayerView * len(self.layers))(*[l.view() for l in self.layers])
            embs = (Q4View * self.num_groups)(*[e.view() for e in self.codec_embeddings])
            heads = (Q4View * self.num_groups)(*[h.view() for h in self.lm_heads])
            c = self.cfg
            v = PredictorView(self.input_proj.view(), self.input_proj_bias.ctypes.data, self.num_groups, embs,
                              len(self.layers), layers, heads, self.final_norm_gamma.ctypes.data, c.hidden,
                              c.heads, c.kv_heads, c.head_dim, c.rope_theta, c.max_position)
            self._keep = (layers, embs, heads, v)
        return self._keep[3]

    @property
    def memory_bytes(self) -> int:
        return (self.input_proj.memory_bytes + 4 * self.input_proj_bias.size +
                sum(e.memory_bytes for e in self.codec_embeddings) + sum(l.memory_bytes for l in self.layers) +
                sum(h.memory_bytes for h in self.lm_heads) + 2 * self.final_norm_gamma.size)


# ---------------------------------------------------------------------------
# Device objects
# ---------------------------------------------------------------------------
TEXT_VOCAB_1P7B = 151936  # Qwen3 text vocab: covers the TTS special tokens (151671-151673)

# Special tokens, src/generate_new.rs:24-36.
IM_START, ASSISTANT, NEWLINE = 151644, 77091, 198
TTS_PAD, TTS_BOS, TTS_EOS = 151671, 151672, 151673
CODEC_THINK, CODEC_THINK_BOS, CODEC_THINK_EOS = 2154, 2156, 2157


class TextWeights:
    """Seeded random-init text embedding + two-layer text projection of
    TalkerWeights (src/talker.rs:33-56): text_embedding [text_vocab]
    [text_hidden], fc1 [text_hidden][text_hidden] + bias, fc2 [text_hidden]
    [hidden] + bias, Q4 like the other weights."""

    def __init__(self, seed: int, text_vocab: int = TEXT_VOCAB_1P7B, text_hidden: int = 2048, hidden: int = 2048):
        self.text_vocab, self.text_hidden, self.hidden = text_vocab, text_hidden, hidden
        self.text_embedding = Q4Weight.synthetic(seed, "text.embedding", text_vocab, text_hidden)
        self.fc1 = Q4Weight.synthetic(seed, "text.fc1", text_hidden, text_hidden)
        self.fc1_bias = synth_normal_f32(seed, "text.fc1_bias", text_hidden, 0.0, 0.02)
        self.fc2 = Q4Weight.synthetic(seed, "text.fc2", text_hidden, hidden)
        self.fc2_bias = synth_normal_f32(seed, "text.fc2_bias", hidden, 0.0, 0.02)

    def view(self) -> "TextView":
        return TextView(self.text_embedding.view(), self.fc1.view(), self.fc1_bias.ctypes.data, self.fc2.view(),
                        self.fc2_bias.ctypes.data, self.text_hidden)


def _f32(a, n: Optional[int] = None) -> np.ndarray:
    a = np.ascontiguousarray(a, dtype=np.float32)
    if n is not None and a.size < n:
        raise ValueError(f"expected at least {n} floats, got {a.size}")
    return a


# ---------------------------------------------------------------------------
# Speech decoder weights (SpeechDecoderWeights, src/decoder.rs:22-65)
# ---------------------------------------------------------------------------
@dataclasses.dataclass
class DecoderConfig:
    hidden: int = 512
    heads: int = 16
    head_dim: int = 64
    inter: int = 1024
    window: int = 72
    codebook_dim: int = 256
    codebook_size: int = 2048
    vq_dim: int = 512
    latent: int = 1024
    num_rest: int = 15
    layers: int = 8
    upsample: tuple = (2, 2)  # ConvNeXt stage strides (transposed kernel = stride)
    convnext_kernel: int = 7
    convnext_mult: int = 4
    vocos_channels: int = 1536
    vocos: tuple = ((1536, 768, 16, 8), (768, 384, 10, 5), (384, 192, 8, 4), (192, 96, 6, 3))  # in, out, k, stride
    dilations: tuple = (1, 3, 9)
    res_kernel: int = 7
    out_kernel: int = 7
    rope_rows: int = 8000
    rope_theta: float = 10000.0


# The 12 Hz tokenizer's decoder (src/loader.rs:503-718).
DECODER_1P7B = DecoderConfig()


class DecoderWeights:
    """Random-init SpeechDecoderWeights of a DecoderConfig (weights scaled by
    1/sqrt(fan-in) so the signal keeps its size through the stack)."""

    def __init__(self, seed: int, cfg: DecoderConfig = DECODER_1P7B):
        self.cfg = c = cfg
        self.seed = seed
        self._arrays = []
        n = lambda name, count, std, mean=0.0: self._keep(synth_normal_f32(seed, f"dec.{name}", count, mean, std))
        cd, vq, lat, hid = c.codebook_dim, c.vq_dim, c.latent, c.hidden
        ad = c.heads * c.head_dim
        self.first_codebook = n("cb0", c.codebook_size * cd, 0.5)
        self.first_output_proj = n("cb0.proj", cd * vq, cd ** -0.5)
        self.rest_codebooks = [n(f"cb{g + 1}", c.codebook_size * cd, 0.5 / 4) for g in range(c.num_rest)]
        self.rest_output_proj = n("cbr.proj", cd * vq, cd ** -0.5)
        self.convs = {}
        self.pre_conv = self._conv("pre_conv", vq, lat, 3, 1, 0, 1)
        self.tf_input_w = n("tf.in.w", lat * hid, lat ** -0.5)
        self.tf_input_b = n("tf.in.b", hid, 0.02)
        self.layers = []
        for i in range(c.layers):
            p = f"tf.{i}"
            self.layers.append(dict(
                q_proj=n(p + ".q", hid * ad, hid ** -0.5), k_proj=n(p + ".k", hid * ad, hid ** -0.5),
                v_proj=n(p + ".v", hid * ad, hid ** -0.5), o_proj=n(p + ".o", ad * hid, ad ** -0.5),
                gate_proj=n(p + ".g", hid * c.inter, hid ** -0.5), up_proj=n(p + ".u", hid * c.inter, hid ** -0.5),
                down_proj=n(p + ".d", c.inter * hid, c.inter ** -0.5),
                input_norm=n(p + ".n1", hid, 0.1, 1.0), post_attn_norm=n(p + ".n2", hid, 0.1, 1.0),
                attn_scale=n(p + ".s1", hid, 0.02, 0.1), mlp_scale=n(p + ".s2", hid, 0.02, 0.1)))
        self.tf_norm = n("tf.norm", hid, 0.1, 1.0)
        self.tf_output_w = n("tf.out.w", hid * lat, hid ** -0.5)
        self.tf_output_b = n("tf.out.b", lat, 0.02)
        self.upsample = []
        for i, s in enumerate(c.upsample):
            p = f"up.{i}"
            inner = lat * c.convnext_mult
            self.upsample.append(dict(
                conv_t=self._conv(p + ".ct", lat, lat, s, s, 0, 1, transposed=True),
                dw_conv=self._dw(p + ".dw", lat, c.convnext_kernel),
                norm_w=n(p + ".nw", lat, 0.1, 1.0), norm_b=n(p + ".nb", lat, 0.02),
                pw1_w=n(p + ".p1w", lat * inner, lat ** -0.5), pw1_b=n(p + ".p1b", inner, 0.02),
                pw2_w=n(p + ".p2w", inner * lat, inner ** -0.5), pw2_b=n(p + ".p2b", lat, 0.02),
                gamma=n(p + ".g", lat, 0.02, 0.1), inner=inner))
        self.vocos_init = self._conv("vocos.init", lat, c.vocos_channels, 7, 1, 0, 1)
        self.blocks = []
        for b, (cin, cout, k, s) in enumerate(c.vocos):
            p = f"vocos.{b}"
            res = []
            for r, d in enumerate(c.dilations):
                q = f"{p}.r{r}"
                res.append(dict(act1_alpha=n(q + ".a1", cout, 0.1), act1_beta=n(q + ".b1", cout, 0.1),
                                conv1=self._conv(q + ".c1", cout, cout, c.res_kernel, 1, 0, d),
                                act2_alpha=n(q + ".a2", cout, 0.1), act2_beta=n(q + ".b2", cout, 0.1),
                                conv2=self._conv(q + ".c2", cout, cout, 1, 1, 0, 1, gain=0.5)))
            self.blocks.append(dict(pre_snake_alpha=n(p + ".sa", cin, 0.1), pre_snake_beta=n(p + ".sb", cin, 0.1),
                                    upsample=self._conv(p + ".up", cin, cout, k, s, 0, 1, transposed=True),
                                    residuals=res))
        last = c.vocos[-1][1] if c.vocos else c.vocos_channels
        self.final_snake_alpha = n("final.a", last, 0.1)
        self.final_snake_beta = n("final.b", last, 0.1)
        self.output_conv = self._conv("out", last, 1, c.out_kernel, 1, 0, 1, gain=0.05)
        half = c.head_dim // 2
        freq = 1.0 / c.rope_theta ** (np.arange(half, dtype=np.float64) * 2 / c.head_dim)
        ang = np.arange(c.rope_rows, dtype=np.float64)[:, None] * freq[None, :]
        self.rope_cos = self._keep(np.cos(ang).astype(np.float32).reshape(-1))
        self.rope_sin = self._keep(np.sin(ang).astype(np.float32).reshape(-1))
        self._view = None

    def _keep(self, a):
        a = np.ascontiguousarray(a, dtype=np.float32)
        self._arrays.append(a)
        return a

    def _conv(self, name, cin, cout, k, stride, pad, dil, transposed=False, gain=1.0):
        """Conv1dWeight [out][in][k] or ConvTranspose1dWeight [in][out][k]."""
        fan = cin * (max(1, k // stride) if transposed else k)
        w = self._keep(synth_normal_f32(self.seed, f"dec.{name}.w", cin * cout * k, 0.0, gain * fan ** -0.5))
        b = self._keep(synth_normal_f32(self.seed, f"dec.{name}.b", cout, 0.0, 0.02))
        return dict(weight=w, bias=b, in_channels=cin, out_channels=cout, kernel_size=k, stride=stride,
                    padding=pad, dilation=dil)

    def _dw(self, name, ch, k):
        w = self._keep(synth_normal_f32(self.seed, f"dec.{name}.w", ch * k, 0.0, k ** -0.5))
        b = self._keep(synth_normal_f32(self.seed, f"dec.{name}.b", ch, 0.0, 0.02))
        return dict(weight=w, bias=b, in_channels=ch, out_channels=ch, kernel_size=k, stride=1,
                    padding=(k - 1) // 2, dilation=1)

    @staticmethod
    def _cv(d) -> ConvView:
        return ConvView(d["weight"].ctypes.data, d["bias"].ctypes.data, d["in_channels"], d["out_channels"],
                        d["kernel_size"], d["stride"], d["padding"], d["dilation"])

    def view(self) -> DecoderView:
        if self._view is not None:
            return self._view[0]
        c = self.cfg
        ptr = lambda a: a.ctypes.data
        rest = (C.c_void_p * c.num_rest)(*[ptr(a) for a in self.rest_codebooks])
        layers = (DecLayerView * len(self.layers))(*[DecLayerView(*[ptr(L[n]) for n, _ in DecLayerView._fields_])
                                                      for L in self.layers])
        ups = (UpsampleView * len(self.upsample))(*[UpsampleView(
            u["conv_t"]["in_channels"], u["inner"], self._cv(u["conv_t"]), self._cv(u["dw_conv"]),
            *[ptr(u[n]) for n in ("norm_w", "norm_b", "pw1_w", "pw1_b", "pw2_w", "pw2_b", "gamma")])
            for u in self.upsample])
        res_arrays = []
        blocks = []
        for b in self.blocks:
            ra = (VocosResidualView * len(b["residuals"]))(*[VocosResidualView(
                ptr(r["act1_alpha"]), ptr(r["act1_beta"]), self._cv(r["conv1"]), ptr(r["act2_alpha"]),
                ptr(r["act2_beta"]), self._cv(r["conv2"])) for r in b["residuals"]])
            res_arrays.append(ra)
            blocks.append(VocosBlockView(ptr(b["pre_snake_alpha"]), ptr(b["pre_snake_beta"]),
                                         self._cv(b["upsample"]), len(b["residuals"]), ra))
        barr = (VocosBlockView * len(blocks))(*blocks)
        v = DecoderView(c.hidden, c.heads, c.head_dim, c.inter, c.window, c.codebook_dim, c.codebook_size, c.vq_dim,
                        ptr(self.first_codebook), ptr(self.first_output_proj), c.num_rest, rest,
                        ptr(self.rest_output_proj), self._cv(self.pre_conv), ptr(self.tf_input_w),
                        ptr(self.tf_input_b), len(self.layers), layers, ptr(self.tf_norm), ptr(self.tf_output_w),
                        ptr(self.tf_output_b), len(self.upsample), ups, self._cv(self.vocos_init), len(blocks), barr,
                        ptr(self.final_snake_alpha), ptr(self.final_snake_beta), self._cv(self.output_conv),
                        ptr(self.rope_cos), ptr(self.rope_sin), c.rope_rows)
        self._view = (v, rest, layers, ups, res_arrays, barr)
        return v

    def synthetic_codes(self, seed: int, frames: int) -> np.ndarray:
        """[num_rest + 1][frames] codes below codebook_size."""
        raw = np.empty(frames * (self.cfg.num_rest + 1), dtype=np.float32)
        load_library().qtts_synth_normal_f32(seed, stream_id("dec.codes"), raw.size, 0.0, 1.0, _ptr(raw))
        u = (np.abs(raw.astype(np.float64)) * 1e6).astype(np.int64) % self.cfg.codebook_size
        return u.astype(np.uint32).reshape(self.cfg.num_rest + 1, frames)


class SpeechDecoder(_DeviceObject):
    """SpeechDecoderWeights in HBM with decode_to_audio."""

    _free_fn = "qtts_decoder_free"

    def __init__(self, ctx: "Context", w):
        self.cfg = getattr(w, "cfg", None)
        h = C.c_void_p()
        self._view = w.view()
        ctx.check(ctx.lib.qtts_decoder_upload(ctx.h, C.byref(self._view), C.byref(h)))
        self._register(ctx, h)

    def num_samples(self, frames: int) -> int:
        return int(self.ctx.lib.qtts_decoder_num_samples(self.h, frames))

    # decode_to_audio, src/decoder.rs:394-509
    def decode_to_audio(self, codes) -> np.ndarray:
        codes = np.ascontiguousarray(codes, dtype=np.uint32)
        groups, frames = codes.shape
        out = np.empty(max(1, self.num_samples(frames)), dtype=np.float32)
        n = C.c_int64()
        self.ctx.check(self.ctx.lib.qtts_decode_to_audio(self.h, _ptr(codes), frames, frames, _ptr(out), out.size,
                                                         C.byref(n)))
        return out[: n.value]

    def decode_to_audio_device(self, d_codes: int, frames: int, ld: int, d_audio: int, capacity: int) -> int:
        n = C.c_int64()
        self.ctx.check(self.ctx.lib.qtts_decode_to_audio_device(self.h, C.c_void_p(d_codes), frames, ld,
                                                                C.c_void_p(d_audio), capacity, C.byref(n)))
        return n.value


# ---------------------------------------------------------------------------
# .qora-tts model files (load_model, src/save.rs:262-298)
# ---------------------------------------------------------------------------
def q4_from_view(v: Q4View) -> Q4Weight:
    """A host copy of a Q4 view's arrays."""
    packed = np.ctypeslib.as_array(C.cast(v.packed, C.POINTER(C.c_uint8)), (v.k * v.n // 2,)).copy()
    scales = np.ctypeslib.as_array(C.cast(v.scales, C.POINTER(C.c_uint16)), (v.k * v.n // 32,)).copy()
    return Q4Weight(packed, scales, v.k, v.n)


class _FileStack:
    """A talker or predictor section of an open model file, usable wherever
    TalkerWeights / CodePredictorWeights are (it has .cfg and .view())."""

    def __init__(self, owner, view, cfg, **extra):
        self._owner, self._view, self.cfg = owner, view, cfg
        self.__dict__.update(extra)

    def view(self):
        return self._view


class ModelFile:
    """An opened .qora-tts file: .talker, .predictor (upload-ready views with
    the file's RoPE tables), .text (the prompt-assembly weights) and .info."""

    def __init__(self, path: str):
        lib = load_library()
        h = C.c_void_p()
        rc = lib.qtts_model_file_open(os.fsencode(path), C.byref(h))
        if rc != QTTS_OK:
            raise QttsError(rc, lib.qtts_model_file_error().decode())
        self.h, self._lib = h, lib
        tv = lib.qtts_model_file_talker(h).contents
        pv = lib.qtts_model_file_predictor(h).contents
        self.info = lib.qtts_model_file_info(h).contents
        self.text = lib.qtts_model_file_text(h).contents
        l0 = tv.layers[0]
        tcfg = StackConfig(layers=tv.num_layers, hidden=tv.hidden_size, heads=tv.num_heads,
                           kv_heads=tv.num_kv_heads, head_dim=tv.head_dim, inter=l0.gate_proj.n,
                           vocab=tv.codec_head.n, max_position=tv.max_position, rope_theta=0.0)
        p0 = pv.layers[0]
        pcfg = StackConfig(layers=pv.num_layers, hidden=pv.hidden_size, heads=pv.num_heads,
                           kv_heads=pv.num_kv_heads, head_dim=pv.head_dim, inter=p0.gate_proj.n,
                           vocab=pv.lm_heads[0].n, max_position=pv.max_position, rope_theta=0.0)
        dv = lib.qtts_model_file_decoder(h).contents
        self.decoder = _FileStack(self, dv, None)
        self.talker = _FileStack(self, tv, tcfg)
        self.predictor = _FileStack(self, pv, pcfg, num_groups=pv.num_groups,
                                    talker_hidden=pv.codec_embeddings[0].n)

    def close(self):
        if getattr(self, "h", None):
            self._lib.qtts_model_file_close(self.h)
            self.h = None

    def __del__(self):
        self.close()


class Context:
    """One HIP device + stream (qtts_ctx)."""

    def __init__(self, device: int = 0):
        self.lib = load_library()
        self._children = weakref.WeakSet()  # device objects made from this context
        h = C.c_void_p()
        st = self.lib.qtts_ctx_create(device, C.byref(h))
        if st != QTTS_OK:
            raise QttsError(st, f"qtts_ctx_create(device={device}) failed")
        self.h = h

    def check(self, st: int):
        if st != QTTS_OK:
            raise QttsError(st, self.lib.qtts_last_error(self.h).decode())

    @property
    def stream(self) -> int:
        return self.lib.qtts_ctx_stream(self.h)

    def synchronize(self):
        self.check(self.lib.qtts_ctx_synchronize(self.h))

    def close(self):
        """Frees every object made from this context that is still open, then
        the context: all device memory and the stream are released here, while
        the HIP runtime is up, rather than by finalizers at interpreter exit."""
        if getattr(self, "h", None):
            try:
                self.synchronize()
            except QttsError:
                pass  # the objects are freed all the same
            for obj in list(self._children):
                obj.close()
            self.lib.qtts_ctx_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    # sample_token, src/generate_new.rs:329-391
    def sample_token(self, logits, temperature=0.8, top_k=50, repetition_penalty=1.05, prev_tokens=(0,) * 16,
                     rng: int = 0, greedy: bool = False):
        """Returns (token, new_rng_state)."""
        lg = _f32(logits)
        prev = np.ascontiguousarray(prev_tokens, dtype=np.uint32)
        p = SamplerParams(temperature, top_k, repetition_penalty, 1 if greedy else 0)
        state = C.c_uint64(rng)
        tok = C.c_uint32(0)
        self.check(self.lib.qtts_sample_token(self.h, _ptr(lg), lg.size, C.byref(p), _ptr(prev), prev.size,
                                              C.byref(state), C.byref(tok)))
        return int(tok.value), int(state.value)

    # sample_top_k of the legacy generator, src/generate.rs:50-84
    def sample_top_k(self, logits, temperature: float, top_k: int, rng: int = 0):
        """Returns (token, new_rng_state)."""
        lg = _f32(logits)
        state = C.c_uint64(rng)
        tok = C.c_uint32(0)
        self.check(self.lib.qtts_sample_top_k(self.h, _ptr(lg), lg.size, float(temperature), int(top_k),
                                              C.byref(state), C.byref(tok)))
        return int(tok.value), int(state.value)


class DeviceQ4(_DeviceObject):
    """A Weight::Q4 resident in HBM with gemv/gemm/embed_lookup (src/gemv.rs:148-176)."""

    _free_fn = "qtts_q4_free"

    def __init__(self, ctx: Context, w: Q4Weight):
        self.k, self.n = w.k, w.n
        h = C.c_void_p()
        v = w.view()
        ctx.check(ctx.lib.qtts_q4_upload(ctx.h, C.byref(v), C.byref(h)))
        self._register(ctx, h)

    def gemv(self, x) -> np.ndarray:
        x = _f32(x, self.k)
        y = np.empty(self.n, dtype=np.float32)
        self.ctx.check(self.ctx.lib.qtts_gemv(self.ctx.h, self.h, _ptr(x), _ptr(y)))
        return y

    def gemm(self, x, seq_len: int) -> np.ndarray:
        x = _f32(x, seq_len * self.k)
        y = np.empty(seq_len * self.n, dtype=np.float32)
        self.ctx.check(self.ctx.lib.qtts_gemm(self.ctx.h, self.h, _ptr(x), seq_len, _ptr(y)))
        return y

    def embed_lookup(self, token: int) -> np.ndarray:
        y = np.empty(self.n, dtype=np.float32)
        self.ctx.check(self.ctx.lib.qtts_embed_lookup(self.ctx.h, self.h, int(token), _ptr(y)))
        return y

    def gemv_device(self, d_x: int, d_y: int):
        self.ctx.check(self.ctx.lib.qtts_gemv_device(self.ctx.h, self.h, C.c_void_p(d_x), C.c_void_p(d_y)))

    def gemm_device(self, d_x: int, seq_len: int, d_y: int):
        """gemm over device buffers (x: seq_len rows of K, y: seq_len rows of N)."""
        self.ctx.check(self.ctx.lib.qtts_gemm_device(self.ctx.h, self.h, C.c_void_p(d_x), seq_len, C.c_void_p(d_y)))

    @property
    def memory_bytes(self) -> int:
        return int(self.ctx.lib.qtts_q4_bytes(self.h))


class KvCache(_DeviceObject):
    """RawKvCache (src/gemv.rs:75-86) in HBM, fixed capacity."""

    _free_fn = "qtts_kv_free"

    def __init__(self, ctx: Context, num_layers: int, num_kv_heads: int, head_dim: int, capacity: int):
        self.shape = (num_layers, num_kv_heads, head_dim)
        h = C.c_void_p()
        ctx.check(ctx.lib.qtts_kv_create(ctx.h, num_layers, num_kv_heads, head_dim, capacity, C.byref(h)))
        self._register(ctx, h)

    def __len__(self) -> int:
        return int(self.ctx.lib.qtts_kv_len(self.h))

    def clear(self):
        self.ctx.check(self.ctx.lib.qtts_kv_clear(self.h))

    def load(self, k: np.ndarray, v: np.ndarray, length: int):
        """k, v: [layers][length][kv_heads][head_dim] float32."""
        k, v = _f32(k), _f32(v)
        self.ctx.check(self.ctx.lib.qtts_kv_load(self.h, _ptr(k), _ptr(v), length))

    def store(self):
        L, H, D = self.shape
        n = len(self)
        k = np.empty((L, n, H, D), dtype=np.float32)
        v = np.empty_like(k)
        self.ctx.check(self.ctx.lib.qtts_kv_store(self.h, _ptr(k), _ptr(v)))
        return k, v


class Talker(_DeviceObject):
    """TalkerWeights in HBM with the reference's talker functions."""

    _free_fn = "qtts_talker_free"

    def __init__(self, ctx: Context, w: TalkerWeights):
        self.cfg = w.cfg
        h = C.c_void_p()
        v = w.view()
        ctx.check(ctx.lib.qtts_talker_upload(ctx.h, C.byref(v), C.byref(h)))
        self._register(ctx, h)

    def new_kv(self, capacity: int) -> KvCache:
        c = self.cfg
        return KvCache(self.ctx, c.layers, c.kv_heads, c.head_dim, capacity)

    # forward_with_embedding, src/talker.rs:263-360
    def forward_with_embedding(self, embedding, kv: KvCache, position: int) -> np.ndarray:
        e = _f32(embedding, self.cfg.hidden)
        out = np.empty(self.cfg.hidden + self.cfg.vocab, dtype=np.float32)
        self.ctx.check(self.ctx.lib.qtts_forward_with_embedding(self.h, _ptr(e), kv.h, position, _ptr(out)))
        return out

    # prefill_talker_raw, src/talker.rs:364-462
    def prefill_talker_raw(self, x, seq_len: int, kv: KvCache) -> np.ndarray:
        x = _f32(x, seq_len * self.cfg.hidden)
        out = np.empty(self.cfg.hidden, dtype=np.float32)
        self.ctx.check(self.ctx.lib.qtts_prefill_talker_raw(self.h, _ptr(x), seq_len, kv.h, _ptr(out)))
        return out

    # prefill_talker, src/talker.rs:467-488: (token, is_text) rows
    def prefill_talker(self, tokens, is_text, kv: KvCache) -> np.ndarray:
        t = np.ascontiguousarray(tokens, dtype=np.uint32)
        f = np.ascontiguousarray(np.asarray(is_text, dtype=bool), dtype=np.int32)
        if t.shape != f.shape:
            raise ValueError("tokens and is_text differ in length")
        out = np.empty(self.cfg.hidden, dtype=np.float32)
        self.ctx.check(self.ctx.lib.qtts_prefill_talker(self.h, _ptr(t) if t.size else None,
                                                        _ptr(f) if f.size else None, t.size, kv.h, _ptr(out)))
        return out

    # apply_codec_head, src/talker.rs:627-629
    def apply_codec_head(self, hidden) -> np.ndarray:
        hs = _f32(hidden, self.cfg.hidden)
        out = np.empty(self.cfg.vocab, dtype=np.float32)
        self.ctx.check(self.ctx.lib.qtts_apply_codec_head(self.h, _ptr(hs), _ptr(out)))
        return out

    # embed_codec_token, src/talker.rs:152-154
    def embed_codec_token(self, token: int) -> np.ndarray:
        out = np.empty(self.cfg.hidden, dtype=np.float32)
        self.ctx.check(self.ctx.lib.qtts_embed_codec_token(self.h, int(token), _ptr(out)))
        return out

    # forward_talker_decode, src/talker.rs:161-258
    def forward_talker_decode(self, token: int, is_text: bool, kv: KvCache, position: int) -> np.ndarray:
        out = np.empty(self.cfg.hidden, dtype=np.float32)
        self.ctx.check(self.ctx.lib.qtts_forward_talker_decode(self.h, int(token), 1 if is_text else 0, kv.h,
                                                                int(position), _ptr(out)))
        return out

    def attach_text(self, text: "TextWeights"):
        """Uploads the text embedding and projection (qtts_talker_text_upload)."""
        self._text_view = text.view()
        self.ctx.check(self.ctx.lib.qtts_talker_text_upload(self.h, C.byref(self._text_view)))

    # embed_text_token, src/talker.rs:105-116
    def embed_text_token(self, token: int) -> np.ndarray:
        out = np.empty(self.cfg.hidden, dtype=np.float32)
        self.ctx.check(self.ctx.lib.qtts_embed_text_token(self.h, int(token), _ptr(out)))
        return out

    def build_custom_voice_prompt(self, text_tokens, speaker_id: int, language_id: int, voice_embedding=None):
        """The rows prefill_custom_voice runs (src/generate_new.rs:60-177), [L][hidden]."""
        tok = np.ascontiguousarray(text_tokens, dtype=np.uint32)
        voice = None if voice_embedding is None else _f32(voice_embedding, self.cfg.hidden)
        rows = np.empty((10, self.cfg.hidden), dtype=np.float32)
        n = C.c_int32(0)
        self.ctx.check(self.ctx.lib.qtts_build_custom_voice_prompt(self.h, _ptr(tok) if tok.size else None, tok.size,
                                                                    speaker_id, language_id, _ptr(voice), _ptr(rows),
                                                                    C.byref(n)))
        return rows[: n.value].copy()

    # prefill_custom_voice, src/generate_new.rs:84-188
    def prefill_custom_voice(self, text_tokens, speaker_id: int, language_id: int, kv: "KvCache",
                             voice_embedding=None):
        """Returns (last_hidden, logits, position)."""
        tok = np.ascontiguousarray(text_tokens, dtype=np.uint32)
        voice = None if voice_embedding is None else _f32(voice_embedding, self.cfg.hidden)
        lh = np.empty(self.cfg.hidden, dtype=np.float32)
        lg = np.empty(self.cfg.vocab, dtype=np.float32)
        pos = C.c_int32(0)
        self.ctx.check(self.ctx.lib.qtts_prefill_custom_voice(self.h, _ptr(tok) if tok.size else None, tok.size,
                                                               speaker_id, language_id, _ptr(voice), kv.h, _ptr(lh),
                                                               _ptr(lg), C.byref(pos)))
        return lh, lg, pos.value

    # build_trailing_text, src/generate_new.rs:314-326
    def build_trailing_text(self, text_tokens) -> np.ndarray:
        tok = np.ascontiguousarray(text_tokens, dtype=np.uint32)
        rows = np.empty((max(tok.size, 1), self.cfg.hidden), dtype=np.float32)
        n = C.c_int32(0)
        self.ctx.check(self.ctx.lib.qtts_build_trailing_text(self.h, _ptr(tok) if tok.size else None, tok.size,
                                                              _ptr(rows), C.byref(n)))
        return rows[: n.value].copy()


class CodePredictor(_DeviceObject):
    """CodePredictorWeights in HBM with generate_acoustic_codes."""

    _free_fn = "qtts_predictor_free"

    def __init__(self, ctx: Context, w: CodePredictorWeights):
        self.cfg, self.num_groups = w.cfg, w.num_groups
        self.talker_hidden = w.talker_hidden
        h = C.c_void_p()
        v = w.view()
        ctx.check(ctx.lib.qtts_predictor_upload(ctx.h, C.byref(v), C.byref(h)))
        self._register(ctx, h)

    def new_kv(self, capacity: int = 16) -> KvCache:
        c = self.cfg
        return KvCache(self.ctx, c.layers, c.kv_heads, c.head_dim, capacity)

    # generate_acoustic_codes, src/code_predictor.rs:218-273
    def generate_acoustic_codes(self, talker_hidden, semantic_embed, kv: KvCache) -> np.ndarray:
        th = _f32(talker_hidden, self.talker_hidden)
        se = _f32(semantic_embed, self.talker_hidden)
        codes = np.empty(self.num_groups, dtype=np.uint32)
        self.ctx.check(self.ctx.lib.qtts_generate_acoustic_codes(self.h, _ptr(th), _ptr(se), kv.h, _ptr(codes)))
        return codes

    # get_acoustic_embeddings_sum, src/code_predictor.rs:280-293
    def get_acoustic_embeddings_sum(self, codes) -> np.ndarray:
        cs = np.ascontiguousarray(codes, dtype=np.uint32)
        out = np.empty(self.talker_hidden, dtype=np.float32)
        self.ctx.check(self.ctx.lib.qtts_get_acoustic_embeddings_sum(self.h, _ptr(cs), _ptr(out)))
        return out

    # predict_codes, src/code_predictor.rs:126-213
    def predict_codes(self, talker_hidden, kv: KvCache) -> np.ndarray:
        th = _f32(talker_hidden, self.talker_hidden)
        out = np.empty((self.num_groups, self.cfg.vocab), dtype=np.float32)
        self.ctx.check(self.ctx.lib.qtts_predict_codes(self.h, _ptr(th), kv.h, _ptr(out)))
        return out


def loop_params(max_codes: int, temperature: float = 0.8, top_k: int = 50, repetition_penalty: float = 1.05,
                greedy: bool = False, stop_on_eos: bool = True, talker_only: bool = False,
                codec_eos_id: int = CODEC_EOS) -> LoopParams:
    return LoopParams(max_codes, SamplerParams(temperature, top_k, repetition_penalty, 1 if greedy else 0),
                      codec_eos_id, 1 if stop_on_eos else 0, 1 if talker_only else 0)


def generate_codes(talker: Talker, predictor: Optional[CodePredictor], talker_kv: KvCache,
                   predictor_kv: Optional[KvCache], last_hidden, logits, position: int,
                   trailing_text: Optional[np.ndarray], tts_pad_embed: Optional[np.ndarray], params: LoopParams,
                   seed: int) -> np.ndarray:
    """The frame loop of generate_speech (src/generate_new.rs:229-300) on the
    device.  Returns all_codes as [16][n_frames] uint32."""
    ctx = talker.ctx
    hidden = talker.cfg.hidden
    lh = _f32(last_hidden, hidden)
    lg = _f32(logits, talker.cfg.vocab)
    tt = None if trailing_text is None else _f32(trailing_text).reshape(-1, hidden)
    tl = 0 if tt is None else tt.shape[0]
    pad = None if tts_pad_embed is None else _f32(tts_pad_embed, hidden)
    codes = np.zeros((16, max(params.max_codes, 1)), dtype=np.uint32)
    n = C.c_int32(0)
    ctx.check(ctx.lib.qtts_generate_codes(talker.h, predictor.h if predictor is not None else None,
                                          talker_kv.h, predictor_kv.h if predictor_kv is not None else None, _ptr(lh), _ptr(lg),
                                          position, _ptr(tt), tl, _ptr(pad), C.byref(params), seed, _ptr(codes),
                                          C.byref(n)))
    return codes[:, : n.value].copy()


def generate_speech(talker: Talker, predictor: Optional[CodePredictor], decoder: SpeechDecoder, text_tokens,
                    speaker_id: int, language_id: int, talker_kv: KvCache, predictor_kv: Optional[KvCache],
                    params: LoopParams, seed: int, voice_embedding=None):
    """generate_speech (src/generate_new.rs:191-311) from token ids to audio in
    one call; the codes stay in device memory between the frame loop and the
    decoder.  Returns (audio float32, n_frames)."""
    ctx = talker.ctx
    tok = np.ascontiguousarray(text_tokens, dtype=np.uint32)
    voice = None if voice_embedding is None else _f32(voice_embedding, talker.cfg.hidden)
    out = np.empty(max(1, decoder.num_samples(max(params.max_codes, 0))), dtype=np.float32)
    n, nf = C.c_int64(0), C.c_int32(0)
    ctx.check(ctx.lib.qtts_generate_speech(talker.h, predictor.h if predictor is not None else None, decoder.h,
                                           _ptr(tok) if tok.size else None, tok.size, speaker_id, language_id,
                                           _ptr(voice), talker_kv.h,
                                           predictor_kv.h if predictor_kv is not None else None, C.byref(params),
                                           seed, _ptr(out), out.size, C.byref(n), C.byref(nf)))
    return out[: n.value].copy(), nf.value


def generate_speech_codes(talker: Talker, predictor: Optional[CodePredictor], text_tokens, speaker_id: int,
                          language_id: int, talker_kv: KvCache, predictor_kv: Optional[KvCache], params: LoopParams,
                          seed: int, voice_embedding=None) -> np.ndarray:
    """generate_speech (src/generate_new.rs:191-300) from token ids to codes on
    the device: prefill_custom_voice, build_trailing_text, the frame loop.
    Returns all_codes as [16][n_frames] uint32."""
    ctx = talker.ctx
    tok = np.ascontiguousarray(text_tokens, dtype=np.uint32)
    voice = None if voice_embedding is None else _f32(voice_embedding, talker.cfg.hidden)
    codes = np.zeros((16, max(params.max_codes, 1)), dtype=np.uint32)
    n = C.c_int32(0)
    ctx.check(ctx.lib.qtts_generate_speech_codes(talker.h, predictor.h if predictor is not None else None,
                                                 _ptr(tok) if tok.size else None, tok.size, speaker_id, language_id,
                                                 _ptr(voice), talker_kv.h,
                                                 predictor_kv.h if predictor_kv is not None else None,
                                                 C.byref(params), seed, _ptr(codes), C.byref(n)))
    return codes[:, : n.value].copy()


def generate_codes_batch(talker: Talker, predictor: Optional[CodePredictor], talker_kvs, last_hidden, logits,
                         positions, trailing_text: Optional[np.ndarray], tts_pad_embed: Optional[np.ndarray],
                         params: LoopParams, seeds) -> list:
    """len(talker_kvs) independent frame loops in lockstep (one row per
    stream on the matrix cores).  last_hidden [B][hidden], logits [B][vocab],
    trailing_text [B][n][hidden] or None.  Returns each stream's codes as
    [16][n_frames] uint32."""
    ctx = talker.ctx
    B, hidden, vocab = len(talker_kvs), talker.cfg.hidden, talker.cfg.vocab
    lh = _f32(last_hidden, B * hidden)
    lg = _f32(logits, B * vocab)
    tt = None if trailing_text is None else _f32(trailing_text).reshape(B, -1, hidden)
    tl = 0 if tt is None else tt.shape[1]
    pad = None if tts_pad_embed is None else _f32(tts_pad_embed, hidden)
    pos = np.ascontiguousarray(positions, dtype=np.int32)
    sd = np.ascontiguousarray(seeds, dtype=np.uint64)
    kvs = (C.c_void_p * B)(*[kv.h for kv in talker_kvs])
    mc = max(params.max_codes, 1)
    codes = np.zeros((B, 16, mc), dtype=np.uint32)
    n = np.zeros(B, dtype=np.int32)
    ctx.check(ctx.lib.qtts_generate_codes_batch(talker.h, predictor.h if predictor is not None else None, B, kvs,
                                                _ptr(lh), _ptr(lg), _ptr(pos), _ptr(tt), tl, _ptr(pad),
                                                C.byref(params), _ptr(sd), _ptr(codes), _ptr(n)))
    return [codes[b, :, : n[b]].copy() for b in range(B)]
