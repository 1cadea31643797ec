"""ctypes binding of libgrx.so (include/grx.h).

The library is built in-tree (python -m gorelaxor_amd.build); loading it
never falls back to anything else: a missing or unloadable library raises.
"""
from __future__ import annotations

import ctypes as C
import os
import re

PKG = os.path.dirname(os.path.abspath(__file__))
# GRX_LIB names another build of the library (an experiment); default in-tree
LIB_PATH = os.environ.get("GRX_LIB") or os.path.join(PKG, "libgrx.so")
HEADER = os.path.join(os.path.dirname(PKG), "include", "grx.h")

GRX_OK = 0
STATUS = {0: "GRX_OK", -1: "GRX_EINVAL", -2: "GRX_ESIZE", -3: "GRX_EDEVICE", -4: "GRX_ENOMEM",
          -5: "GRX_ESTATE", -6: "GRX_ENODEV"}


class GrxError(RuntimeError):
    """A non-zero grx_status, with grx_last_error()'s message."""

    def __init__(self, status: int, message: str):
        super().__init__(f"{STATUS.get(status, status)}: {message}")
        self.status = status


_lib = None

vp = C.c_void_p
i32 = C.c_int
sz = C.c_size_t

# name -> (restype, argtypes); every grx_* entry point of include/grx.h
SIGNATURES = {
    "grx_version": (i32, []),
    "grx_last_error": (C.c_char_p, []),
    "grx_device_count": (i32, []),
    "grx_ctx_create": (i32, [i32, C.POINTER(vp)]),
    "grx_ctx_destroy": (i32, [vp]),
    "grx_ctx_sync": (i32, [vp]),
    "grx_ctx_stream": (vp, [vp]),
    "grx_weight_q8_create": (i32, [vp, i32, i32, vp, sz, C.POINTER(vp)]),
    "grx_weight_destroy": (i32, [vp]),
    "grx_weight_rows": (i32, [vp]),
    "grx_weight_cols": (i32, [vp]),
    "grx_weight_bytes": (sz, [vp]),
    "grx_weight_row": (i32, [vp, vp, i32, vp]),
    "grx_weight_float32": (i32, [vp, vp, vp]),
    "grx_to_q8": (i32, [vp, i32, i32, vp, vp]),
    "grx_matmul_q8": (i32, [vp, vp, i32, vp, i32, i32, vp, vp]),
    "grx_linear_q8": (i32, [vp, vp, vp, i32, vp, vp]),
    "grx_matmul_q8_dev": (i32, [vp, vp, i32, vp, i32, i32, vp, vp]),
    "grx_matmul_q8_dev_noalloc": (i32, [vp, vp, i32, vp, i32, i32, vp, vp]),
    "grx_quant_act_dev": (i32, [vp, vp, vp, vp, i32, i32, i32]),
    "grx_matmul_q8_prequant_dev": (i32, [vp, vp, i32, vp, vp, i32, vp, vp]),
    "grx_block_dots_dev": (i32, [vp, vp, vp, i32, vp]),
    "grx_vec_dev": (i32, [vp, i32, vp, vp, i32]),
    "grx_layernorm_dev": (i32, [vp, i32, i32, i32, vp, vp, i32, i32, vp, vp, C.c_double]),
    "grx_linear_q8_float": (i32, [vp, vp, vp, vp, vp]),
    "grx_linear_f32": (i32, [vp, vp, vp, vp, i32, i32, vp]),
    "grx_whisper_create": (i32, [vp, vp, C.POINTER(vp)]),
    "grx_whisper_destroy": (i32, [vp]),
    "grx_whisper_set_tensor": (i32, [vp, C.c_char_p, vp, sz]),
    "grx_whisper_set_encoder_output": (i32, [vp, vp, i32]),
    "grx_whisper_reset": (i32, [vp]),
    "grx_whisper_pos": (i32, [vp]),
    "grx_whisper_decode": (i32, [vp, vp, i32, vp, vp]),
    "grx_whisper_greedy": (i32, [vp, vp, i32, i32, vp]),
    "grx_whisper_create_streams": (i32, [vp, vp, i32, C.POINTER(vp)]),
    "grx_whisper_streams": (i32, [vp]),
    "grx_whisper_set_encoder_output_stream": (i32, [vp, i32, vp, i32]),
    "grx_whisper_greedy_streams": (i32, [vp, vp, i32, i32, vp]),
    "grx_whisper_stream_copy": (i32, [vp, i32, i32]),
    "grx_whisper_share_encoder_output": (i32, [vp, i32, i32]),
    "grx_whisper_steps": (i32, [vp, i32, vp]),
    "grx_whisper_logits": (i32, [vp, i32, vp]),
    "grx_whisper_rules_loop": (i32, [vp, vp, vp, vp, vp]),
    "grx_whisper_load_ggml": (i32, [vp, C.c_char_p, i32, vp, C.POINTER(vp)]),
    "grx_whisper_sample_logits": (i32, [vp, vp, i32, vp, vp, C.c_float, C.c_float, vp]),
    "grx_whisper_sample": (i32, [vp, i32, vp, vp, C.c_float, C.c_float, vp]),
    "grx_gguf_open": (i32, [C.c_char_p, C.POINTER(vp)]),
    "grx_gguf_parse": (i32, [vp, sz, C.POINTER(vp)]),
    "grx_gguf_read_meta": (i32, [C.c_char_p, C.POINTER(vp)]),
    "grx_gguf_close": (i32, [vp]),
    "grx_gguf_version": (i32, [vp]),
    "grx_gguf_n_tensors": (i32, [vp]),
    "grx_gguf_tensor_name": (C.c_char_p, [vp, i32]),
    "grx_gguf_n_keys": (i32, [vp]),
    "grx_gguf_key": (C.c_char_p, [vp, i32]),
    "grx_gguf_has": (i32, [vp, C.c_char_p]),
    "grx_gguf_tensor_info": (i32, [vp, C.c_char_p, C.POINTER(i32), C.POINTER(i32), C.POINTER(C.c_int64)]),
    "grx_gguf_int": (C.c_int64, [vp, C.c_char_p, C.c_int64]),
    "grx_gguf_float": (C.c_double, [vp, C.c_char_p, C.c_double]),
    "grx_gguf_bool": (i32, [vp, C.c_char_p, i32]),
    "grx_gguf_string": (C.c_char_p, [vp, C.c_char_p, C.c_char_p]),
    "grx_gguf_array_len": (C.c_int64, [vp, C.c_char_p]),
    "grx_gguf_array_string": (C.c_char_p, [vp, C.c_char_p, C.c_int64]),
    "grx_gguf_array_float": (C.c_double, [vp, C.c_char_p, C.c_int64]),
    "grx_gguf_array_int": (C.c_int64, [vp, C.c_char_p, C.c_int64]),
    "grx_gguf_float32": (i32, [vp, C.c_char_p, vp, sz]),
    "grx_gguf_weight_shape": (i32, [vp, C.c_char_p, C.POINTER(C.c_int64), C.POINTER(C.c_int64)]),
    "grx_gguf_weight_q8": (i32, [vp, vp, C.c_char_p, C.POINTER(vp)]),
    "grx_pocket_create": (i32, [vp, vp, C.POINTER(vp)]),
    "grx_pocket_load_gguf": (i32, [vp, C.c_char_p, i32, vp, C.POINTER(vp)]),
    "grx_pocket_flow_init": (i32, [vp, i32, i32, i32]),
    "grx_pocket_speak": (i32, [vp, vp, vp, i32, vp, vp]),
    "grx_pocket_destroy": (i32, [vp]),
    "grx_pocket_set_tensor": (i32, [vp, C.c_char_p, vp, sz]),
    "grx_pocket_reset": (i32, [vp]),
    "grx_pocket_pos": (i32, [vp]),
    "grx_pocket_run": (i32, [vp, vp, i32, vp]),
    "grx_pocket_frames": (i32, [vp, vp, i32, vp, vp]),
    "grx_pocket_state_create": (i32, [vp, vp, vp, i32, C.POINTER(vp)]),
    "grx_pocket_load_voice_gguf": (i32, [vp, C.c_char_p, C.POINTER(vp)]),
    "grx_pocket_state_save": (i32, [vp, C.POINTER(vp)]),
    "grx_pocket_set_state": (i32, [vp, vp]),
    "grx_pocket_state_positions": (i32, [vp]),
    "grx_pocket_state_read": (i32, [vp, vp, vp]),
    "grx_pocket_state_destroy": (i32, [vp]),
    "grx_conformer_create": (i32, [vp, vp, C.POINTER(vp)]),
    "grx_conformer_load_gguf": (i32, [vp, C.c_char_p, vp, C.POINTER(vp)]),
    "grx_conformer_destroy": (i32, [vp]),
    "grx_conformer_set_tensor": (i32, [vp, C.c_char_p, vp, sz]),
    "grx_conformer_frames_out": (i32, [vp, i32]),
    "grx_conformer_encode": (i32, [vp, vp, i32, i32, vp, vp, vp]),
    "grx_conformer_encode_dev": (i32, [vp, vp, i32, i32, vp, vp]),
    "grx_debug_fail_alloc_after": (None, [C.c_longlong]),
    "grx_debug_alloc_countdown": (C.c_longlong, []),
    "grx_debug_tune": (i32, [C.c_char_p, i32]),
    "grx_conformer_stream_create": (i32, [vp, i32, i32, C.POINTER(vp)]),
    "grx_conformer_stream_destroy": (i32, [vp]),
    "grx_conformer_stream_geometry": (i32, [vp, vp]),
    "grx_conformer_stream_step": (i32, [vp, vp, i32, vp, vp, vp]),
    "grx_conformer_stream_step_dev": (i32, [vp, vp, i32, vp, vp, vp]),
    "grx_mimi_create": (i32, [vp, vp, C.POINTER(vp)]),
    "grx_mimi_destroy": (i32, [vp]),
    "grx_mimi_set_tensor": (i32, [vp, C.c_char_p, vp, sz]),
    "grx_mimi_reset": (i32, [vp]),
    "grx_mimi_decode": (i32, [vp, vp, i32, vp]),
    "grx_mimi_decode_dev": (i32, [vp, vp, i32, vp]),
    "grx_mimi_samples_per_latent": (i32, [vp]),
    "grx_mimi_load_gguf": (i32, [vp, C.c_char_p, i32, vp, C.POINTER(vp)]),
    "grx_rnnt_create": (i32, [vp, vp, C.POINTER(vp)]),
    "grx_rnnt_destroy": (i32, [vp]),
    "grx_rnnt_load_gguf": (i32, [vp, C.c_char_p, vp, C.POINTER(vp)]),
    "grx_rnnt_set_tensor": (i32, [vp, C.c_char_p, vp, sz]),
    "grx_rnnt_state_create": (i32, [vp, C.POINTER(vp)]),
    "grx_rnnt_state_destroy": (i32, [vp]),
    "grx_rnnt_state_read": (i32, [vp, vp, vp, C.POINTER(C.c_int)]),
    "grx_rnnt_state_write": (i32, [vp, vp, vp, i32]),
    "grx_rnnt_decode": (i32, [vp, vp, i32, i32, vp, i32, vp, i32, C.POINTER(C.c_int)]),
}


class PocketHParams(C.Structure):
    """grx_pocket_hparams."""
    _fields_ = [(n, C.c_int) for n in ("d", "heads", "ff", "n_layer", "max_pos", "ldim")] + [("period", C.c_double)]


class ConformerHParams(C.Structure):
    """grx_conformer_hparams."""
    _fields_ = [(n, C.c_int) for n in ("d", "heads", "layers", "dff", "conv_kernel", "sub_channels", "n_mels",
                                       "xscaling", "conv_ln", "att_chunked", "att_left", "att_right", "conv_left",
                                       "conv_right", "causal_sub", "n_context_choices")] + [
        ("context_choices", (C.c_int * 2) * 8)] + [
        (n, C.c_int) for n in ("pre_encode_cache", "drop_extra", "sampling_frames_first")]


class ConformerStreamGeom(C.Structure):
    """grx_conformer_stream_geom."""
    _fields_ = [(n, C.c_int) for n in ("right", "chunk", "left", "left_chunks", "mel_first", "mel_next", "mel_cache",
                                       "drop", "sample_first")]


class RnntHParams(C.Structure):
    """grx_rnnt_hparams."""
    _fields_ = [(n, C.c_int) for n in ("d", "pred_hidden", "pred_layers", "pred_vocab", "joint_hidden", "joint_act",
                                       "tdt", "n_durations")] + [("durations", C.c_int * 16)] + [
        (n, C.c_int) for n in ("max_symbols", "blank")]


class MimiHParams(C.Structure):
    """grx_mimi_hparams."""
    _fields_ = [(n, C.c_int) for n in ("d", "heads", "ff", "layers", "context", "ldim", "upsample")] + [
        ("period", C.c_double), ("n_ratios", C.c_int), ("ratios", C.c_int * 8)] + [
        (n, C.c_int) for n in ("n_filters", "kernel_size", "residual_kernel_size", "last_kernel_size",
                               "dilation_base", "compress", "n_residual", "max_latents")]


class RnntToken(C.Structure):
    """grx_rnnt_token."""
    _fields_ = [("id", C.c_int), ("frame", C.c_int), ("duration", C.c_int), ("p", C.c_float)]


class WhisperRules(C.Structure):
    """grx_whisper_rules."""
    _fields_ = [(n, C.c_int) for n in ("eot", "sot", "translate", "transcribe", "solm", "prev", "nosp",
                                       "no_timestamps", "beg", "n_lang", "space")] + [
        ("suppress", C.POINTER(C.c_int32)), ("n_suppress", C.c_int), ("n_audio_ctx", C.c_int),
        ("max_initial_ts", C.c_double)]


class WhisperSeq(C.Structure):
    """grx_whisper_seq."""
    _fields_ = [(n, C.c_int) for n in ("n_tokens", "last", "penult", "has_ts", "seek_delta")]


class WhisperToken(C.Structure):
    """grx_whisper_token."""
    _fields_ = [("id", C.c_int), ("tid", C.c_int), ("p", C.c_float), ("plog", C.c_float), ("force_ts", C.c_int)]


class WhisperLoop(C.Structure):
    """grx_whisper_loop."""
    _fields_ = [(n, C.c_int) for n in ("seek", "seek_end", "delta_min", "win_frames", "n_max")] + [
        ("temp", C.c_float), ("r", C.POINTER(C.c_float))]


class WhisperLoopResult(C.Structure):
    """grx_whisper_loop_result."""
    _fields_ = [(n, C.c_int) for n in ("n_tokens", "done", "failed", "result_len", "seek_delta", "has_ts")]


class WhisperHParams(C.Structure):
    """grx_whisper_hparams (whisper/model.go:16-21)."""
    _fields_ = [(n, C.c_int) for n in ("n_vocab", "n_text_ctx", "n_state", "n_head", "n_layer", "n_audio_ctx")]


def header_symbols() -> list[str]:
    """Every function include/grx.h declares."""
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(grx_[a-z0-9_]+)\s*\(", text)))


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is not built: run python -m gorelaxor_amd.build")
        L = C.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            f = getattr(L, name)
            f.restype = res
            f.argtypes = args
        _lib = L
    return _lib


def check(status: int) -> None:
    if status != GRX_OK:
        msg = lib().grx_last_error()
        raise GrxError(status, msg.decode() if msg else "")


def call(name: str, *args) -> None:
    check(getattr(lib(), name)(*args))
