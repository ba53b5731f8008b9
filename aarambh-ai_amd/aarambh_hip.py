"""Python host mirror of aarambh-studio's speculative-verify interface over the
HIP C ABI (include/aarambh_hip.h, libaarambh_hip.so).

The names follow the reference crates so that tests read like the reference's
own:
  ModelConfig / MtpConfig          core/src/config.rs:734-776, 275-283
  Sampler.greedy / top_k_top_p     inference/src/sampler.rs:33-65
  SpeculativeConfig                inference/src/speculative.rs:14-31
  SpeculativeStats                 inference/src/speculative.rs:41-90
  HipModel.forward_with_cache_output / forward_mtp_head
                                   model/src/model.rs:529-587, 783-817
  HipModel KV snapshot / restore   inference/src/kvcache.rs:56-69
  MtpSpeculativeEngine.generate    inference/src/mtp_speculative.rs:86-336
Errors raise AarambhError subclasses (core/src/error.rs:5-33).  There is no
CPU fallback: a missing or unloadable library raises immediately.
"""
import atexit
import collections
import ctypes as C
import os
import weakref
from dataclasses import dataclass, field
from typing import Optional

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libaarambh_hip.so")

W_F32, W_BF16, W_INT8_ROW, W_INT4_G128 = 0, 1, 2, 3
KV_F32, KV_F16, KV_INT8 = 0, 1, 2
T_NORM, T_LINEAR, T_EMBED = 0, 1, 2
FLAG_RATIO_NEAR, FLAG_CDF_NEAR, FLAG_TOPP_NEAR = 1, 2, 8
TOP_CANDIDATES = 5  # engine.rs:70
REPLAY_REPLACEMENT, REPLAY_REFERENCE = 0, 1
PROF_NAMES = ["gemv_qkv", "gemv_wo", "gemv_gateup", "gemv_down", "gemv_lmhead", "attention", "accept", "other"]


class AarambhError(RuntimeError):
    pass


class ConfigError(AarambhError):
    pass


class ShapeError(AarambhError):
    pass


class UnsupportedError(AarambhError):
    pass


class DeviceError(AarambhError):
    pass


class CheckpointError(AarambhError):
    pass


class IoError(AarambhError):
    pass


_ERRS = {1: ConfigError, 2: ShapeError, 3: UnsupportedError, 4: DeviceError, 5: CheckpointError, 6: IoError}


class _Cfg(C.Structure):
    _fields_ = [(n, C.c_int32) for n in ("vocab_size", "hidden_dim", "ffn_dim", "n_layers", "n_heads",
                                          "n_kv_heads", "max_seq_len")] + \
               [("rope_theta", C.c_float), ("norm_eps", C.c_float)] + \
               [(n, C.c_int32) for n in ("num_future_tokens", "weight_format", "lm_head_format", "kv_format",
                                          "max_batch", "max_rows", "untied_lm_head")]


class _RopeScaling(C.Structure):
    _fields_ = [("method", C.c_int32), ("original_max_seq_len", C.c_int32), ("factor", C.c_double),
                ("beta_fast", C.c_double), ("beta_slow", C.c_double), ("attn_factor", C.c_double)]


class _LatCfg(C.Structure):
    _fields_ = [(n, C.c_int32) for n in ("vocab_size", "hidden_dim", "n_layers", "n_heads", "max_seq_len")] + \
               [("rope_theta", C.c_float), ("norm_eps", C.c_float)] + \
               [(n, C.c_int32) for n in ("latent_dim", "rope_dim", "nope_dim", "v_dim", "n_experts", "top_k",
                                          "expert_dim", "n_shared", "expert_format", "attn_format",
                                          "lm_head_format", "kv_format", "max_batch", "max_rows",
                                          "untied_lm_head")]


class _Sampler(C.Structure):
    _fields_ = [("greedy", C.c_int32), ("temperature", C.c_float), ("top_k", C.c_int32), ("top_p", C.c_float)]


class _Stats(C.Structure):
    _fields_ = [(n, C.c_int32) for n in ("rounds", "draft_tokens_proposed", "draft_tokens_accepted",
                                          "draft_tokens_rejected", "target_decode_forwards",
                                          "draft_decode_forwards", "mtp_head_forwards")]


_lib = None
_P = C.c_void_p


def lib():
    """Load libaarambh_hip.so; raises if it is missing (no fallback path)."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise DeviceError(f"HIP library not built: {LIB_PATH} (run __graft_entry__.build())")
    L = C.CDLL(LIB_PATH)
    sig = {
        "aarh_create": (C.c_int, [C.c_int, C.POINTER(_Cfg), C.POINTER(_P)]),
        "aarh_destroy": (None, [_P]),
        "aarh_last_error": (C.c_char_p, [_P]),
        "aarh_stream": (_P, [_P]),
        "aarh_sync": (C.c_int, [_P]),
        "aarh_num_tensors": (C.c_int, [_P]),
        "aarh_tensor_info": (C.c_int, [_P, C.c_int, C.c_char_p, C.c_int, C.POINTER(C.c_int64),
                                       C.POINTER(C.c_int64), C.POINTER(C.c_int32)]),
        "aarh_load_tensor_f32": (C.c_int, [_P, C.c_int, _P, C.c_int64]),
        "aarh_load_tensor_int4": (C.c_int, [_P, C.c_int, _P, _P, _P, C.c_int64, C.c_int64, C.c_int32]),
        "aarh_load_tensor_int8": (C.c_int, [_P, C.c_int, _P, _P, C.c_int64, C.c_int64]),
        "aarh_load_tensor_packed_i4": (C.c_int, [_P, C.c_int, _P, C.c_int32, C.c_int64, _P, C.c_int64, _P, _P,
                                                 C.c_int64]),
        "aarh_lat_load_tensor_packed_i4": (C.c_int, [_P, C.c_int, _P, C.c_int32, C.c_int64, _P, C.c_int64, _P, _P,
                                                     C.c_int64]),
        "aarh_packed_i4_params": (C.c_int, [_P, C.c_int32, C.c_int64, C.c_int64, _P, _P, C.c_int64, _P, _P]),
        "aarh_init_synthetic": (C.c_int, [_P, C.c_uint64, C.c_float]),
        "aarh_get_config": (C.c_int, [_P, C.POINTER(_Cfg)]),
        "aarh_set_replay_schedule": (C.c_int, [_P, C.c_int]),
        "aarh_load_gguf": (C.c_int, [_P, C.c_char_p, C.POINTER(C.c_int32)]),
        "aarh_load_safetensors": (C.c_int, [_P, C.c_char_p, C.POINTER(C.c_int32)]),
        "aarh_gguf_config": (C.c_int, [C.c_char_p, C.POINTER(_Cfg)]),
        "aarh_gguf_read_tensor": (C.c_int, [C.c_char_p, C.c_char_p, _P, C.c_int64, C.POINTER(C.c_int64),
                                            C.POINTER(C.c_int32), C.POINTER(C.c_int64), C.POINTER(C.c_int32)]),
        "aarh_safetensors_read_tensor": (C.c_int, [C.c_char_p, C.c_char_p, _P, C.c_int64, C.POINTER(C.c_int64),
                                                   C.POINTER(C.c_int32), C.POINTER(C.c_int64)]),
        "aarh_host_last_error": (C.c_char_p, []),
        "aarh_kv_reset": (C.c_int, [_P, C.c_int]),
        "aarh_kv_len": (C.c_int, [_P, C.c_int, C.POINTER(C.c_int32)]),
        "aarh_kv_rollback": (C.c_int, [_P, C.c_int, C.c_int32]),
        "aarh_kv_fill_synthetic": (C.c_int, [_P, C.c_int, C.c_int32, C.c_uint64]),
        "aarh_forward": (C.c_int, [_P, _P, _P, _P, C.c_int, C.c_int, _P, _P]),
        "aarh_last_logits_device": (_P, [_P]),
        "aarh_last_hidden_device": (_P, [_P]),
        "aarh_mtp_head": (C.c_int, [_P, C.c_int, _P, _P, C.c_int, _P]),
        "aarh_accept_sample": (C.c_int, [_P, _P, C.c_int, _P, _P, _P, C.c_int, C.c_int, C.c_int, C.c_int,
                                         C.POINTER(_Sampler), _P, _P, _P, _P, _P, _P, _P, _P, _P]),
        "aarh_accept_sample_static": (C.c_int, [_P, _P, C.c_int, _P, _P, _P, C.c_int, C.c_int, C.c_int, C.c_int,
                                                C.POINTER(_Sampler), _P, _P, _P, _P, _P, _P, _P, _P, _P]),
        "aarh_mtp_generate": (C.c_int, [_P, _P, C.c_int, C.c_int, C.c_int, C.c_int, C.POINTER(_Sampler), _P,
                                        _P, _P, _P, C.POINTER(_Stats)]),
        "aarh_session_begin": (C.c_int, [_P, _P, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, C.POINTER(_Sampler),
                                         _P, C.POINTER(_P)]),
        "aarh_session_step": (C.c_int, [_P, C.c_int, C.POINTER(C.c_int32)]),
        "aarh_session_result": (C.c_int, [_P, _P, C.c_int32, _P, _P, C.POINTER(_Stats)]),
        "aarh_session_end": (None, [_P]),
        "aarh_session_open": (C.c_int, [_P, C.c_int, C.c_int, C.POINTER(_Sampler), C.POINTER(_P)]),
        "aarh_session_admit": (C.c_int, [_P, C.c_int, _P, C.c_int, C.c_int, C.c_uint64, C.c_int]),
        "aarh_session_retire": (C.c_int, [_P, C.c_int]),
        "aarh_session_rows": (C.c_int, [_P, _P]),
        "aarh_spec_generate": (C.c_int, [_P, _P, _P, C.c_int, C.c_int, C.c_int, C.c_int, C.POINTER(_Sampler), _P,
                                         _P, _P, _P, C.POINTER(_Stats), _P, _P]),
        "aarh_session_candidates": (C.c_int, [_P, _P, _P, C.c_int32]),
        "aarh_spec_session_begin": (C.c_int, [_P, _P, _P, C.c_int, C.c_int, C.c_int, C.c_int, C.POINTER(_Sampler),
                                              _P, C.POINTER(_P)]),
        "aarh_spec_session_step": (C.c_int, [_P, C.c_int, C.POINTER(C.c_int32)]),
        "aarh_spec_session_result": (C.c_int, [_P, _P, C.c_int32, _P, _P, C.POINTER(_Stats)]),
        "aarh_spec_session_candidates": (C.c_int, [_P, _P, _P, C.c_int32]),
        "aarh_spec_session_rng_offsets": (C.c_int, [_P, _P]),
        "aarh_spec_session_set_rng_offsets": (C.c_int, [_P, _P]),
        "aarh_spec_session_end": (None, [_P]),
        "aarh_session_rng_offsets": (C.c_int, [_P, _P]),
        "aarh_session_set_rng_offsets": (C.c_int, [_P, _P]),
        "aarh_top_candidates": (C.c_int, [_P, _P, C.c_int, C.c_int, C.POINTER(_Sampler), C.c_int, _P, _P, _P]),
        "aarh_set_graphs": (C.c_int, [_P, C.c_int]),
        "aarh_set_rope_scaling": (C.c_int, [_P, C.POINTER(_RopeScaling)]),
        "aarh_gguf_rope_scaling": (C.c_int, [C.c_char_p, C.POINTER(_RopeScaling)]),
        "aarh_prof_enable": (C.c_int, [_P, C.c_int]),
        "aarh_prof_get": (C.c_int, [_P, C.c_int, C.POINTER(C.c_double), C.POINTER(C.c_double),
                                    C.POINTER(C.c_int64)]),
        "aarh_lat_create": (C.c_int, [C.c_int, C.POINTER(_LatCfg), C.POINTER(_P)]),
        "aarh_lat_get_config": (C.c_int, [_P, C.POINTER(_LatCfg)]),
        "aarh_lat_load_gguf": (C.c_int, [_P, C.c_char_p, C.POINTER(C.c_int32)]),
        "aarh_lat_load_safetensors": (C.c_int, [_P, C.c_char_p, C.POINTER(C.c_int32)]),
        "aarh_lat_gguf_config": (C.c_int, [C.c_char_p, C.POINTER(_LatCfg)]),
        "aarh_lat_destroy": (None, [_P]),
        "aarh_lat_last_error": (C.c_char_p, [_P]),
        "aarh_lat_num_tensors": (C.c_int, [_P]),
        "aarh_lat_tensor_info": (C.c_int, [_P, C.c_int, C.c_char_p, C.c_int, C.POINTER(C.c_int64),
                                           C.POINTER(C.c_int64), C.POINTER(C.c_int32)]),
        "aarh_lat_load_tensor_f32": (C.c_int, [_P, C.c_int, _P, C.c_int64]),
        "aarh_lat_init_synthetic": (C.c_int, [_P, C.c_uint64, C.c_float]),
        "aarh_lat_kv_len": (C.c_int, [_P, C.c_int, C.POINTER(C.c_int32)]),
        "aarh_lat_kv_rollback": (C.c_int, [_P, C.c_int, C.c_int32]),
        "aarh_lat_kv_fill_synthetic": (C.c_int, [_P, C.c_int, C.c_int32, C.c_uint64]),
        "aarh_lat_forward": (C.c_int, [_P, _P, _P, _P, C.c_int, C.c_int, _P, _P]),
        "aarh_lat_router_gaps": (C.c_int, [_P, _P]),
        "aarh_lat_expert_counts": (C.c_int, [_P, _P]),
        "aarh_lat_prof_enable": (C.c_int, [_P, C.c_int]),
        "aarh_lat_prof_get": (C.c_int, [_P, C.c_int, C.POINTER(C.c_double), C.POINTER(C.c_double),
                                        C.POINTER(C.c_int64)]),
    }
    for name, (res, args) in sig.items():
        f = getattr(L, name)
        f.restype = res
        f.argtypes = args
    _lib = L
    return L


EXPORTED = ["aarh_create", "aarh_destroy", "aarh_last_error", "aarh_stream", "aarh_sync", "aarh_num_tensors",
            "aarh_tensor_info", "aarh_load_tensor_f32", "aarh_load_tensor_int4", "aarh_load_tensor_int8",
            "aarh_init_synthetic", "aarh_kv_reset", "aarh_kv_len", "aarh_kv_rollback", "aarh_kv_fill_synthetic",
            "aarh_forward", "aarh_last_logits_device", "aarh_last_hidden_device", "aarh_mtp_head",
            "aarh_accept_sample", "aarh_mtp_generate", "aarh_session_begin", "aarh_session_step",
            "aarh_session_result", "aarh_session_end", "aarh_spec_generate", "aarh_prof_enable", "aarh_prof_get",
            "aarh_session_candidates", "aarh_top_candidates", "aarh_set_graphs", "aarh_session_rng_offsets",
            "aarh_session_set_rng_offsets", "aarh_accept_sample_static", "aarh_get_config", "aarh_set_replay_schedule", "aarh_load_gguf",
            "aarh_load_safetensors", "aarh_gguf_config", "aarh_gguf_read_tensor", "aarh_host_last_error",
            "aarh_safetensors_read_tensor", "aarh_session_open", "aarh_session_admit", "aarh_session_retire",
            "aarh_session_rows",
            "aarh_lat_create", "aarh_lat_destroy", "aarh_lat_last_error", "aarh_lat_num_tensors",
            "aarh_lat_tensor_info", "aarh_lat_load_tensor_f32", "aarh_lat_init_synthetic", "aarh_lat_kv_len",
            "aarh_lat_kv_rollback", "aarh_lat_kv_fill_synthetic", "aarh_lat_forward", "aarh_lat_router_gaps",
            "aarh_lat_expert_counts", "aarh_lat_prof_enable", "aarh_lat_prof_get", "aarh_load_tensor_packed_i4",
            "aarh_lat_load_tensor_packed_i4", "aarh_packed_i4_params", "aarh_spec_session_begin",
            "aarh_spec_session_step", "aarh_spec_session_result", "aarh_spec_session_candidates",
            "aarh_spec_session_rng_offsets", "aarh_spec_session_set_rng_offsets", "aarh_spec_session_end",
            "aarh_set_rope_scaling", "aarh_gguf_rope_scaling", "aarh_lat_get_config", "aarh_lat_load_gguf",
            "aarh_lat_load_safetensors", "aarh_lat_gguf_config"]


def _ptr(a):
    return None if a is None else C.c_void_p(a.ctypes.data)


def _host_check(st):
    if st:
        raise _ERRS.get(st, AarambhError)(lib().aarh_host_last_error().decode())


def gguf_read_tensor(path, name):
    """One tensor of a GGUF v1 file decoded to f32 by the library's host reader
    (decode_tensor, weights/src/gguf.rs:143-241).  Returns (values, encoding)."""
    n, nd, enc = C.c_int64(), C.c_int32(), C.c_int32()
    shape = (C.c_int64 * 8)()
    p, nm = os.fsencode(path), name.encode()
    _host_check(lib().aarh_gguf_read_tensor(p, nm, None, 0, C.byref(n), C.byref(nd), shape, C.byref(enc)))
    out = np.empty(n.value, np.float32)
    _host_check(lib().aarh_gguf_read_tensor(p, nm, _ptr(out), out.size, None, None, None, None))
    return out.reshape([shape[i] for i in range(nd.value)]), enc.value


def safetensors_read_tensor(path, name):
    """One tensor of a safetensors file as f32 by the library's host reader."""
    n, nd = C.c_int64(), C.c_int32()
    shape = (C.c_int64 * 8)()
    p, nm = os.fsencode(path), name.encode()
    _host_check(lib().aarh_safetensors_read_tensor(p, nm, None, 0, C.byref(n), C.byref(nd), shape))
    out = np.empty(n.value, np.float32)
    _host_check(lib().aarh_safetensors_read_tensor(p, nm, _ptr(out), out.size, None, None, None))
    return out.reshape([shape[i] for i in range(nd.value)])


@dataclass
class PackedInt4Tensor:
    """quant/src/types.rs:79-90: packed 4-bit codes over the flattened row-major tensor
    (low nibble = even index, int4.rs:45-53), f32 scale and zero point per group of
    `group_size` values; value = (q - zero) * scale (dequantise_packed_i4_to_vec,
    int4.rs:70-91)."""
    shape: tuple
    group_size: int
    data: np.ndarray
    scales: np.ndarray
    zeros: np.ndarray

    def _args(self):
        shape = np.ascontiguousarray(self.shape, np.int64)
        data = np.ascontiguousarray(self.data, np.uint8).reshape(-1)
        sc = np.ascontiguousarray(self.scales, np.float32).reshape(-1)
        zz = np.ascontiguousarray(self.zeros, np.float32).reshape(-1)
        if sc.size != zz.size:
            raise ShapeError(f"got {sc.size} scales and {zz.size} zeros")
        return shape, data, sc, zz


def packed_i4_params(t: PackedInt4Tensor):
    """The device's per-(row, 128-column group) fp16 scale and zero bits of a
    PackedInt4Tensor (aarh_packed_i4_params): (scales_f16, zeros_f16) as uint16 [rows, cols/128]."""
    shape, data, sc, zz = t._args()
    cols = int(shape[-1]) if shape.size else 0
    rows = int(np.prod(shape[:-1])) if shape.size > 1 else 1
    ng = max(rows * (cols // 128), 1)
    sh = np.zeros(ng, np.uint16)
    zh = np.zeros(ng, np.uint16)
    _host_check(lib().aarh_packed_i4_params(_ptr(shape), shape.size, int(t.group_size), data.size, _ptr(sc), _ptr(zz),
                                            sc.size, _ptr(sh), _ptr(zh)))
    return sh.reshape(rows, -1), zh.reshape(rows, -1)


ROPE_METHODS = {"yarn": 1, "ntk": 2, "linear": 3}


@dataclass
class RopeScaling:
    """RopeScalingConfig (core/src/config.rs:19-47; field defaults as its Default impl):
    method "yarn" | "ntk" | "linear"."""
    method: str = "yarn"
    factor: float = 1.0
    original_max_seq_len: int = 0
    beta_fast: float = 32.0
    beta_slow: float = 1.0
    attn_factor: float = 1.0

    def _c(self):
        if self.method not in ROPE_METHODS:
            raise ConfigError(f"unknown rope_scaling method {self.method!r}")
        return _RopeScaling(ROPE_METHODS[self.method], int(self.original_max_seq_len), float(self.factor),
                            float(self.beta_fast), float(self.beta_slow), float(self.attn_factor))


@dataclass
class ModelConfig:
    """ModelConfig subset (core/src/config.rs:734-776) plus MtpConfig.num_future_tokens."""
    vocab_size: int
    hidden_dim: int
    ffn_dim: int
    n_layers: int
    n_heads: int
    n_kv_heads: int
    max_seq_len: int
    rope_theta: float = 10000.0
    norm_eps: float = 1e-5
    num_future_tokens: int = 0
    weight_format: int = W_F32
    lm_head_format: int = 0
    kv_format: int = KV_F32
    tie_embeddings: bool = True
    rope_scaling: Optional[RopeScaling] = None

    @classmethod
    def from_gguf(cls, path, **overrides):
        """Model shape from a GGUF v1 file's config (load_gguf_tensors, gguf.rs:91-125),
        tie_embeddings and rope_scaling included; storage formats come from `overrides`
        (defaults as the dataclass)."""
        c = _Cfg()
        p = os.fsencode(path)
        _host_check(lib().aarh_gguf_config(p, C.byref(c)))
        rs = _RopeScaling()
        _host_check(lib().aarh_gguf_rope_scaling(p, C.byref(rs)))
        scaling = None
        if rs.method:
            name = {v: k for k, v in ROPE_METHODS.items()}[rs.method]
            scaling = RopeScaling(name, rs.factor, rs.original_max_seq_len, rs.beta_fast, rs.beta_slow, rs.attn_factor)
        kw = dict(vocab_size=c.vocab_size, hidden_dim=c.hidden_dim, ffn_dim=c.ffn_dim, n_layers=c.n_layers,
                  n_heads=c.n_heads, n_kv_heads=c.n_kv_heads, max_seq_len=c.max_seq_len, rope_theta=c.rope_theta,
                  norm_eps=c.norm_eps, num_future_tokens=c.num_future_tokens,
                  tie_embeddings=not c.untied_lm_head, rope_scaling=scaling)
        kw.update(overrides)
        return cls(**kw)

    @property
    def head_dim(self):  # core/src/config.rs:866-868
        return self.hidden_dim // self.n_heads


@dataclass
class Sampler:
    """inference/src/sampler.rs:14-65: Greedy, or TopKTopP with temperature, optional
    top_k (0: none) and top_p (outside (0, 1): none) and the StdRng seed."""
    greedy: bool = True
    temperature: float = 1.0
    top_k: int = 0
    top_p: float = 0.0
    seed: int = 0

    @staticmethod
    def greedy_sampler():
        return Sampler(greedy=True)

    @staticmethod
    def top_k_top_p(temperature, top_k=None, top_p=None, seed=0):
        if temperature < 0:
            raise ConfigError("temperature must be non-negative")
        if top_p is not None and not (0.0 <= top_p <= 1.0):
            raise ConfigError("top_p must be in [0, 1]")
        return Sampler(False, temperature, top_k or 0, top_p or 0.0, seed)

    def is_deterministic(self):  # sampler.rs:91-97
        return self.greedy or self.temperature <= np.finfo(np.float32).eps

    def _c(self):
        return _Sampler(1 if self.greedy else 0, self.temperature, self.top_k, self.top_p)


@dataclass
class SpeculativeConfig:
    num_draft_tokens: int = 4

    def __post_init__(self):
        if self.num_draft_tokens == 0:
            raise ConfigError("num_draft_tokens must be greater than zero")


@dataclass
class SpeculativeStats:
    rounds: int = 0
    draft_tokens_proposed: int = 0
    draft_tokens_accepted: int = 0
    draft_tokens_rejected: int = 0
    target_decode_forwards: int = 0
    draft_decode_forwards: int = 0
    mtp_head_forwards: int = 0

    def acceptance_rate(self):
        return 0.0 if self.draft_tokens_proposed == 0 else self.draft_tokens_accepted / self.draft_tokens_proposed

    def accepted_tokens_per_target_forward(self):
        return 0.0 if self.target_decode_forwards == 0 else self.draft_tokens_accepted / self.target_decode_forwards


@dataclass
class GenerationOutput:
    token_ids: list
    finish_reason: str
    speculative_stats: SpeculativeStats = field(default_factory=SpeculativeStats)
    # per committed token: [(token_id, probability)] * TOP_CANDIDATES (GenerationStep.candidates,
    # engine.rs:95-110); filled by Session.result and SpeculativeEngine
    candidates: list = field(default_factory=list)


FINISH = {0: "MaxTokens", 1: "EosToken", 2: "ContextLimit"}


def _candidate_lists(ids, probs):
    return [[(int(i), float(p)) for i, p in zip(ri, rp)] for ri, rp in zip(ids, probs)]


_LIVE = weakref.WeakSet()


@atexit.register
def _close_live_contexts():
    # Destroy contexts while the HIP runtime is still up (its own teardown runs later).
    for m in list(_LIVE):
        m.close()


class HipModel:
    """Device copy of one target model plus its KV cache slots."""

    def __init__(self, cfg: ModelConfig, max_batch=1, max_rows=128, device=0):
        self.cfg = cfg
        c = _Cfg(cfg.vocab_size, cfg.hidden_dim, cfg.ffn_dim, cfg.n_layers, cfg.n_heads, cfg.n_kv_heads,
                 cfg.max_seq_len, cfg.rope_theta, cfg.norm_eps, cfg.num_future_tokens, cfg.weight_format,
                 cfg.lm_head_format, cfg.kv_format, max_batch, max_rows, 0 if cfg.tie_embeddings else 1)
        h = _P()
        st = lib().aarh_create(device, C.byref(c), C.byref(h))
        self.h = h
        if st:
            msg = lib().aarh_last_error(h).decode() if h else "aarh_create failed"
            self.close()
            raise _ERRS.get(st, AarambhError)(msg)
        if cfg.rope_scaling is not None:
            try:
                self.set_rope_scaling(cfg.rope_scaling)
            except AarambhError:
                self.close()
                raise
        self.max_batch = max_batch
        self.max_rows = max_rows
        _LIVE.add(self)

    def close(self):
        if getattr(self, "h", None):
            lib().aarh_destroy(self.h)
            self.h = None

    def __del__(self):
        self.close()

    def _check(self, st):
        if st:
            raise _ERRS.get(st, AarambhError)(lib().aarh_last_error(self.h).decode())

    def tensors(self):
        out = []
        name = C.create_string_buffer(128)
        for i in range(lib().aarh_num_tensors(self.h)):
            r, c, k = C.c_int64(), C.c_int64(), C.c_int32()
            self._check(lib().aarh_tensor_info(self.h, i, name, 128, C.byref(r), C.byref(c), C.byref(k)))
            out.append((name.value.decode(), r.value, c.value, k.value))
        return out

    def load_f32(self, tid, values):
        v = np.ascontiguousarray(values, np.float32)
        self._check(lib().aarh_load_tensor_f32(self.h, tid, _ptr(v), v.size))

    def load_int4(self, tid, packed, scales_f16, zeros_f16, rows, cols, group=128):
        p = np.ascontiguousarray(packed, np.uint8)
        s = np.ascontiguousarray(scales_f16, np.uint16)
        z = np.ascontiguousarray(zeros_f16, np.uint16)
        self._check(lib().aarh_load_tensor_int4(self.h, tid, _ptr(p), _ptr(s), _ptr(z), rows, cols, group))

    def load_packed_i4(self, tid, t: PackedInt4Tensor):
        """A PackedInt4Tensor as the quant crate holds it (aarh_load_tensor_packed_i4)."""
        shape, data, sc, zz = t._args()
        self._check(lib().aarh_load_tensor_packed_i4(self.h, tid, _ptr(shape), shape.size, int(t.group_size),
                                                     _ptr(data), data.size, _ptr(sc), _ptr(zz), sc.size))

    def load_int8(self, tid, codes, scales, rows, cols):
        q = np.ascontiguousarray(codes, np.int8)
        s = np.ascontiguousarray(scales, np.float32)
        self._check(lib().aarh_load_tensor_int8(self.h, tid, _ptr(q), _ptr(s), rows, cols))

    def load_gguf(self, path):
        """Loads every tensor of a GGUF v1 checkpoint (load_gguf, gguf.rs:82-89); returns the count."""
        n = C.c_int32()
        self._check(lib().aarh_load_gguf(self.h, os.fsencode(path), C.byref(n)))
        return n.value

    def load_safetensors(self, path):
        """Loads a safetensors checkpoint (load_model_with_dtype, weights/src/lib.rs:68-79)."""
        n = C.c_int32()
        self._check(lib().aarh_load_safetensors(self.h, os.fsencode(path), C.byref(n)))
        return n.value

    def init_synthetic(self, seed=0, std=0.02):
        self._check(lib().aarh_init_synthetic(self.h, seed, std))

    # --- KV cache (inference/src/kvcache.rs) ---
    def kv_len(self, slot=0):
        v = C.c_int32()
        self._check(lib().aarh_kv_len(self.h, slot, C.byref(v)))
        return v.value

    def kv_reset(self, slot=0):
        self._check(lib().aarh_kv_reset(self.h, slot))

    def snapshot(self, slot=0):
        return self.kv_len(slot)

    def restore(self, snapshot, slot=0):
        self._check(lib().aarh_kv_rollback(self.h, slot, snapshot))

    def kv_fill_synthetic(self, slot, length, seed=0):
        self._check(lib().aarh_kv_fill_synthetic(self.h, slot, length, seed))

    # --- model API ---
    def forward_with_cache_output(self, ids, offsets, slots=None, want_logits=True, want_hidden=True):
        """ids [nseq, S]; returns (logits [nseq, S, V], hidden [nseq, S, H])."""
        ids = np.ascontiguousarray(np.atleast_2d(ids), np.uint32)
        nseq, S = ids.shape
        offs = np.ascontiguousarray(np.broadcast_to(np.asarray(offsets, np.int32), (nseq,)), np.int32)
        sl = np.ascontiguousarray(np.arange(nseq, dtype=np.int32) if slots is None else slots, np.int32)
        lg = np.empty((nseq, S, self.cfg.vocab_size), np.float32) if want_logits else None
        hd = np.empty((nseq, S, self.cfg.hidden_dim), np.float32) if want_hidden else None
        self._check(lib().aarh_forward(self.h, _ptr(ids), _ptr(sl), _ptr(offs), nseq, S, _ptr(lg), _ptr(hd)))
        return lg, hd

    def forward_mtp_head(self, head, anchor, ids):
        anchor = np.ascontiguousarray(np.atleast_2d(anchor), np.float32)
        ids = np.ascontiguousarray(np.atleast_2d(ids), np.uint32)
        nseq = anchor.shape[0]
        out = np.empty((nseq, self.cfg.vocab_size), np.float32)
        self._check(lib().aarh_mtp_head(self.h, head, _ptr(anchor), _ptr(ids), nseq, _ptr(out)))
        return out

    def sync(self):
        self._check(lib().aarh_sync(self.h))

    def stream(self):
        return lib().aarh_stream(self.h)

    def set_replay_schedule(self, schedule):
        """REPLAY_REPLACEMENT (default) or REPLAY_REFERENCE (mtp_speculative.rs:302-313)."""
        self._check(lib().aarh_set_replay_schedule(self.h, int(schedule)))

    def set_rope_scaling(self, scaling: Optional[RopeScaling]):
        """RopeCache::from_config with rope_scaling (rope_scaling.rs:24-92); None: unscaled."""
        self._check(lib().aarh_set_rope_scaling(self.h, None if scaling is None else C.byref(scaling._c())))
        self.rope_scaling = scaling

    def set_graphs(self, on=True):
        """Replay captured HIP graphs for repeated verify-forward shapes (default on)."""
        self._check(lib().aarh_set_graphs(self.h, 1 if on else 0))

    def prof_enable(self, on=True):
        self._check(lib().aarh_prof_enable(self.h, 1 if on else 0))

    def prof_get(self):
        out = {}
        for i, n in enumerate(PROF_NAMES):
            ms, by, cnt = C.c_double(), C.c_double(), C.c_int64()
            self._check(lib().aarh_prof_get(self.h, i, C.byref(ms), C.byref(by), C.byref(cnt)))
            out[n] = {"ms": ms.value, "bytes": by.value, "launches": cnt.value}
        return out

    def top_candidates(self, logits, sampler, n=TOP_CANDIDATES):
        """Sampler::top_candidates_from_probabilities of each row of a device logits tensor
        [rows, V] (torch, f32) under `sampler`; returns (ids [rows, n] int32, probs [rows, n])."""
        import torch
        rows, V = logits.shape
        ids = torch.empty((rows, n), dtype=torch.int32, device=logits.device)
        probs = torch.empty((rows, n), dtype=torch.float32, device=logits.device)
        torch.cuda.synchronize()
        self._check(lib().aarh_top_candidates(self.h, C.c_void_p(logits.data_ptr()), rows, V,
                                              C.byref(sampler._c()), n, C.c_void_p(ids.data_ptr()),
                                              C.c_void_p(probs.data_ptr()), None))
        self.sync()
        return ids, probs

    def accept_sample(self, target, draft, draft_tokens, sampler, bonus, seeds=None, word_offsets=None,
                      uniforms=None, n_proposals=None, no_alloc=False):
        """Acceptance on device tensors (torch cuda tensors).  target [B, Kt, V] f32,
        draft [B, K, V] f32, draft_tokens [B, K] int32.  Returns a dict of torch tensors.
        no_alloc=True calls aarh_accept_sample_static (statically allocated scratch)."""
        import torch
        B, K, V = draft.shape if draft is not None else (target.shape[0], 0, target.shape[2])
        dev = target.device
        outs = {k: torch.empty(B, dtype=torch.int32, device=dev)
                for k in ("accept_len", "token", "flags", "draws", "status")}

        def p(t):
            return None if t is None else C.c_void_p(t.data_ptr())

        torch.cuda.synchronize(dev)
        fn = lib().aarh_accept_sample_static if no_alloc else lib().aarh_accept_sample
        st = fn(self.h, p(target), target.shape[1], p(draft), p(draft_tokens), p(n_proposals), B, K, V,
                1 if bonus else 0, C.byref(sampler._c()), p(seeds), p(word_offsets), p(uniforms),
                p(outs["accept_len"]), p(outs["token"]), p(outs["flags"]), p(outs["draws"]), p(outs["status"]),
                None)
        self._check(st)
        self.sync()
        return outs


class MtpSpeculativeEngine:
    """inference/src/mtp_speculative.rs:18-336 for a batch of independent requests."""

    def __init__(self, model: HipModel, config: SpeculativeConfig):
        mtp = model.cfg.num_future_tokens
        if mtp < 2:
            raise ConfigError("internal speculative decoding requires model.mtp configuration")
        if config.num_draft_tokens < 2:
            raise ConfigError("MTP speculative decoding requires at least two proposal tokens")
        if config.num_draft_tokens > mtp:
            raise ConfigError(f"requested {config.num_draft_tokens} MTP proposal tokens but checkpoint horizon is {mtp}")
        self.model = model
        self.config = config

    def generate_batch(self, prompts, max_new_tokens, sampler: Sampler, seeds=None):
        prompts = np.ascontiguousarray(np.atleast_2d(prompts), np.uint32)
        nseq, plen = prompts.shape
        sd = np.ascontiguousarray(
            np.full(nseq, sampler.seed, np.uint64) if seeds is None else seeds, np.uint64)
        out = np.zeros((nseq, max(max_new_tokens, 1)), np.uint32)
        n = np.zeros(nseq, np.int32)
        fin = np.zeros(nseq, np.int32)
        stats = (_Stats * nseq)()
        m = self.model
        m._check(lib().aarh_mtp_generate(m.h, _ptr(prompts), nseq, plen, max_new_tokens,
                                         self.config.num_draft_tokens, C.byref(sampler._c()), _ptr(sd),
                                         _ptr(out), _ptr(n), _ptr(fin), stats))
        res = []
        for b in range(nseq):
            st = SpeculativeStats(**{k: getattr(stats[b], k) for k, _ in _Stats._fields_})
            res.append(GenerationOutput(list(out[b, :n[b]]), FINISH[int(fin[b])], st))
        return res

    def generate(self, prompt_ids, max_new_tokens, sampler: Sampler):
        return self.generate_batch(np.asarray(prompt_ids)[None, :], max_new_tokens, sampler)[0]

    def session(self, prompts, max_new_tokens, sampler: Sampler, cached_len=0, seeds=None):
        return Session(self, prompts, max_new_tokens, sampler, cached_len, seeds)


class SpeculativeEngine:
    """inference/src/speculative.rs:93-516: external draft model speculation for a
    batch of independent requests (target and draft are two HipModels on one device)."""

    def __init__(self, target: HipModel, draft: HipModel, config: SpeculativeConfig):
        if config.num_draft_tokens == 0:
            raise ConfigError("num_draft_tokens must be greater than zero")
        if target.cfg.vocab_size != draft.cfg.vocab_size:
            raise ConfigError("draft and target tokenizers are incompatible (vocabulary sizes differ)")
        self.target = target
        self.draft = draft
        self.config = config

    def generate_batch(self, prompts, max_new_tokens, sampler: Sampler, seeds=None):
        prompts = np.ascontiguousarray(np.atleast_2d(prompts), np.uint32)
        nseq, plen = prompts.shape
        sd = np.ascontiguousarray(
            np.full(nseq, sampler.seed, np.uint64) if seeds is None else seeds, np.uint64)
        out = np.zeros((nseq, max(max_new_tokens, 1)), np.uint32)
        n = np.zeros(nseq, np.int32)
        fin = np.zeros(nseq, np.int32)
        stats = (_Stats * nseq)()
        cap = max(max_new_tokens, 1)
        ci = np.zeros((nseq, cap, TOP_CANDIDATES), np.uint32)
        cp = np.zeros((nseq, cap, TOP_CANDIDATES), np.float32)
        t = self.target
        t._check(lib().aarh_spec_generate(t.h, self.draft.h, _ptr(prompts), nseq, plen, max_new_tokens,
                                          self.config.num_draft_tokens, C.byref(sampler._c()), _ptr(sd),
                                          _ptr(out), _ptr(n), _ptr(fin), stats, _ptr(ci), _ptr(cp)))
        res = []
        for b in range(nseq):
            st = SpeculativeStats(**{k: getattr(stats[b], k) for k, _ in _Stats._fields_})
            res.append(GenerationOutput(list(out[b, :n[b]]), FINISH[int(fin[b])], st,
                                        _candidate_lists(ci[b, :n[b]], cp[b, :n[b]])))
        return res

    def generate(self, prompt_ids, max_new_tokens, sampler: Sampler):
        return self.generate_batch(np.asarray(prompt_ids)[None, :], max_new_tokens, sampler)[0]

    def session(self, prompts, max_new_tokens, sampler: Sampler, seeds=None):
        return SpecSession(self, prompts, max_new_tokens, sampler, seeds)


class SpecSession:
    """Round-by-round driver of the external-draft engine (aarh_spec_session_*)."""

    def __init__(self, engine, prompts, max_new_tokens, sampler, seeds=None):
        self.engine = engine
        t = engine.target
        prompts = np.ascontiguousarray(np.atleast_2d(prompts), np.uint32)
        self.nseq = prompts.shape[0]
        self.max_new = max_new_tokens
        sd = np.ascontiguousarray(
            np.full(self.nseq, sampler.seed, np.uint64) if seeds is None else seeds, np.uint64)
        h = _P()
        t._check(lib().aarh_spec_session_begin(t.h, engine.draft.h, _ptr(prompts), self.nseq, prompts.shape[1],
                                               max_new_tokens, engine.config.num_draft_tokens,
                                               C.byref(sampler._c()), _ptr(sd), C.byref(h)))
        self.h = h

    def step(self, rounds=1):
        done = C.c_int32()
        self.engine.target._check(lib().aarh_spec_session_step(self.h, rounds, C.byref(done)))
        return bool(done.value)

    def result(self):
        cap = max(self.max_new, 1)
        n = self.nseq
        out = np.zeros((n, cap), np.uint32)
        ln = np.zeros(n, np.int32)
        fin = np.zeros(n, np.int32)
        stats = (_Stats * n)()
        t = self.engine.target
        t._check(lib().aarh_spec_session_result(self.h, _ptr(out), cap, _ptr(ln), _ptr(fin), stats))
        ci = np.zeros((n, cap, TOP_CANDIDATES), np.uint32)
        cp = np.zeros((n, cap, TOP_CANDIDATES), np.float32)
        t._check(lib().aarh_spec_session_candidates(self.h, _ptr(ci), _ptr(cp), cap))
        res = []
        for b in range(n):
            st = SpeculativeStats(**{k: getattr(stats[b], k) for k, _ in _Stats._fields_})
            res.append(GenerationOutput(list(out[b, :ln[b]]), FINISH[int(fin[b])], st,
                                        _candidate_lists(ci[b, :ln[b]], cp[b, :ln[b]])))
        return res

    def rng_offsets(self):
        out = np.zeros(self.nseq, np.uint64)
        self.engine.target._check(lib().aarh_spec_session_rng_offsets(self.h, _ptr(out)))
        return out

    def set_rng_offsets(self, offsets):
        o = np.ascontiguousarray(offsets, np.uint64)
        self.engine.target._check(lib().aarh_spec_session_set_rng_offsets(self.h, _ptr(o)))

    def close(self):
        if getattr(self, "h", None):
            lib().aarh_spec_session_end(self.h)
            self.h = None

    def __del__(self):
        self.close()


def _session_outputs(model, h, n, cap, candidates=True):
    """GenerationOutput of every row of a session (committed tokens up to `cap` per row)."""
    cap = max(cap, 1)
    out = np.zeros((n, cap), np.uint32)
    ln = np.zeros(n, np.int32)
    fin = np.zeros(n, np.int32)
    stats = (_Stats * n)()
    model._check(lib().aarh_session_result(h, _ptr(out), cap, _ptr(ln), _ptr(fin), stats))
    if candidates:
        ci = np.zeros((n, cap, TOP_CANDIDATES), np.uint32)
        cp = np.zeros((n, cap, TOP_CANDIDATES), np.float32)
        model._check(lib().aarh_session_candidates(h, _ptr(ci), _ptr(cp), cap))
    res = []
    for b in range(n):
        st = SpeculativeStats(**{k: getattr(stats[b], k) for k, _ in _Stats._fields_})
        cands = _candidate_lists(ci[b, :ln[b]], cp[b, :ln[b]]) if candidates else []
        res.append(GenerationOutput(list(out[b, :ln[b]]), FINISH[int(fin[b])], st, cands))
    return res


class Session:
    """Round-by-round driver of the MTP engine (aarh_session_*)."""

    def __init__(self, engine, prompts, max_new_tokens, sampler, cached_len=0, seeds=None):
        self.engine = engine
        m = engine.model
        prompts = np.ascontiguousarray(np.atleast_2d(prompts), np.uint32)
        self.nseq = prompts.shape[0]
        self.max_new = max_new_tokens
        sd = np.ascontiguousarray(
            np.full(self.nseq, sampler.seed, np.uint64) if seeds is None else seeds, np.uint64)
        h = _P()
        m._check(lib().aarh_session_begin(m.h, _ptr(prompts), self.nseq, prompts.shape[1], cached_len,
                                          max_new_tokens, engine.config.num_draft_tokens, C.byref(sampler._c()),
                                          _ptr(sd), C.byref(h)))
        self.h = h

    def step(self, rounds=1):
        done = C.c_int32()
        self.engine.model._check(lib().aarh_session_step(self.h, rounds, C.byref(done)))
        return bool(done.value)

    def result(self):
        return _session_outputs(self.engine.model, self.h, self.nseq, self.max_new)

    def rng_offsets(self):
        """Keystream word position of each request's sampler (the next uniform it draws)."""
        out = np.zeros(self.nseq, np.uint64)
        self.engine.model._check(lib().aarh_session_rng_offsets(self.h, _ptr(out)))
        return out

    def set_rng_offsets(self, offsets):
        o = np.ascontiguousarray(offsets, np.uint64)
        self.engine.model._check(lib().aarh_session_set_rng_offsets(self.h, _ptr(o)))

    def close(self):
        if getattr(self, "h", None):
            lib().aarh_session_end(self.h)
            self.h = None

    def __del__(self):
        self.close()


class ContinuousSession:
    """Row-level driver of the MTP engine for continuous batching (aarh_session_open /
    _admit / _retire / _rows): a request joins a free row between rounds with its own
    prompt, token budget and seed (prepare_session_with_chunk_size, engine.rs:271-317)
    and leaves when it completes or is cancelled; the rounds run every generating row."""

    FREE, GENERATING, FINISHED = 0, 1, 2

    def __init__(self, engine, capacity, sampler: Sampler):
        self.engine = engine
        self.capacity = capacity
        self.budget = [0] * capacity
        h = _P()
        engine.model._check(lib().aarh_session_open(engine.model.h, capacity, engine.config.num_draft_tokens,
                                                    C.byref(sampler._c()), C.byref(h)))
        self.h = h

    def admit(self, row, prompt_ids, max_new_tokens, seed=0, prefill_chunk=128):
        p = np.ascontiguousarray(np.asarray(prompt_ids).reshape(-1), np.uint32)
        self.engine.model._check(lib().aarh_session_admit(self.h, row, _ptr(p), p.size, max_new_tokens, seed,
                                                          prefill_chunk))
        self.budget[row] = max_new_tokens

    def retire(self, row):
        self.engine.model._check(lib().aarh_session_retire(self.h, row))
        self.budget[row] = 0

    def rows(self):
        st = np.zeros(self.capacity, np.int32)
        self.engine.model._check(lib().aarh_session_rows(self.h, _ptr(st)))
        return st

    def step(self, rounds=1):
        done = C.c_int32()
        self.engine.model._check(lib().aarh_session_step(self.h, rounds, C.byref(done)))
        return bool(done.value)

    def results(self, candidates=True):
        return _session_outputs(self.engine.model, self.h, self.capacity, max(self.budget), candidates)

    def close(self):
        if getattr(self, "h", None):
            lib().aarh_session_end(self.h)
            self.h = None

    def __del__(self):
        self.close()


@dataclass
class BatcherConfig:
    """serve/src/batching.rs:18-40 (batch_wait has no counterpart: step() is driven by the
    caller)."""
    max_batch_size: int = 8
    queue_capacity: int = 128
    prefill_chunk_size: int = 128


@dataclass
class GenerationRequest:
    """One request (batching.rs:42-51) as token ids (the tokenizer is not on this path):
    its token budget and its sampler seed (the sampler settings are the batcher's)."""
    prompt_ids: object
    max_new_tokens: int
    seed: int = 0


class QueueFull(AarambhError):
    """SubmitError::QueueFull (batching.rs:66-73)."""


class SpeculativeBatcher:
    """Continuous batching with speculative rounds: one step() is one iteration of the
    serving worker (run_worker, serve/src/batching.rs:324-445) with its single-token
    batched decode (decode_sessions, inference/src/engine.rs:323-355) replaced by MTP
    speculative rounds over the active requests:
      1. admit queued requests in submission order while fewer than max_batch_size are
         active (admit_job, :463-483): a request whose prefill fails is answered with a
         failure and takes no row;
      2. drop requests whose caller cancelled them (:363-367);
      3. run `rounds` speculative rounds over every active request;
      4. report each active request's newly committed tokens, and complete and free the
         requests that finished (:405-432).
    step() returns the events of the iteration in that order: ("delta", id, token_ids),
    ("completed", id, GenerationOutput), ("failed", id, message)."""

    def __init__(self, engine: MtpSpeculativeEngine, config: BatcherConfig, sampler: Sampler, session=None):
        if config.max_batch_size == 0 or config.queue_capacity == 0 or config.prefill_chunk_size == 0:
            raise ConfigError("batch size and queue capacity must be greater than zero")
        self.config = config
        # `session`: an object with ContinuousSession's methods (admit, retire, rows, step,
        # results, close) to drive instead of a new device session
        self.session = session if session is not None else ContinuousSession(engine, config.max_batch_size, sampler)
        self.queue = collections.deque()
        self.active = {}  # row -> [request id, tokens reported]
        self.cancelled = set()
        self.next_id = 0

    def submit(self, request: GenerationRequest):
        if len(self.queue) >= self.config.queue_capacity:
            raise QueueFull("request queue is full")
        rid = self.next_id
        self.next_id += 1
        self.queue.append((rid, request))
        return rid

    def cancel(self, rid):
        self.cancelled.add(rid)

    def pending(self):
        return len(self.queue) + len(self.active)

    def step(self, rounds=1):
        events = []
        free = [b for b in range(self.config.max_batch_size) if b not in self.active]
        while self.queue and free:
            rid, req = self.queue.popleft()
            if rid in self.cancelled:
                self.cancelled.discard(rid)
                continue
            row = free[0]
            try:
                self.session.admit(row, req.prompt_ids, req.max_new_tokens, req.seed,
                                   self.config.prefill_chunk_size)
            except AarambhError as exc:
                events.append(("failed", rid, str(exc)))
                continue
            free.pop(0)
            self.active[row] = [rid, 0]
        for row, (rid, _) in list(self.active.items()):
            if rid in self.cancelled:
                self.cancelled.discard(rid)
                self.session.retire(row)
                del self.active[row]
        if not self.active:
            return events
        try:
            self.session.step(rounds)
        except AarambhError as exc:
            # a failed batched decode fails every active request and frees its row; the
            # batcher keeps serving the queue (run_worker, batching.rs:441-450)
            msg = str(exc)
            for row in sorted(self.active):
                events.append(("failed", self.active[row][0], msg))
                self.session.retire(row)
            self.active.clear()
            return events
        state = self.session.rows()
        done = [row for row in self.active if state[row] == ContinuousSession.FINISHED]
        outs = self.session.results(candidates=bool(done))
        for row in sorted(self.active):
            rid, seen = self.active[row]
            toks = outs[row].token_ids
            if len(toks) > seen:
                events.append(("delta", rid, [int(t) for t in toks[seen:]]))
                self.active[row][1] = len(toks)
        for row in done:
            events.append(("completed", self.active[row][0], outs[row]))
            self.session.retire(row)
            del self.active[row]
        return events

    def run(self, rounds=1):
        """Steps until every submitted request has completed, failed or been cancelled;
        returns the events in order."""
        events = []
        while self.queue or self.active:
            events += self.step(rounds)
        return events

    def close(self):
        self.session.close()


# ---------------------------------------------------------------------------
# Latent-attention MoE decoder (benchmark config 5)
# ---------------------------------------------------------------------------
@dataclass
class LatConfig:
    """MLA (nn/src/mla.rs:300-489) + fine-grained MoE (nn/src/moe.rs:127-406) decoder shape."""
    vocab_size: int
    hidden_dim: int
    n_layers: int
    n_heads: int
    max_seq_len: int
    latent_dim: int = 512
    rope_dim: int = 64
    nope_dim: int = 128
    v_dim: int = 128
    n_experts: int = 64
    top_k: int = 6
    expert_dim: int = 1408
    n_shared: int = 2
    expert_format: int = W_INT4_G128
    attn_format: int = W_INT4_G128
    lm_head_format: int = W_BF16
    kv_format: int = KV_F16
    rope_theta: float = 10000.0
    norm_eps: float = 1e-5
    tie_embeddings: bool = True  # False: an lm_head.weight of its own (LmHead::untied_with_qat)

    @classmethod
    def from_gguf(cls, path, **overrides):
        """Latent shape from a GGUF v1 file's config (aarh_lat_gguf_config: MlaConfig::resolve,
        MoE fine experts, tie_embeddings, the reference's config checks); formats from
        `overrides`."""
        c = _LatCfg()
        _host_check(lib().aarh_lat_gguf_config(os.fsencode(path), C.byref(c)))
        kw = {f: getattr(c, f) for f in ("vocab_size", "hidden_dim", "n_layers", "n_heads", "max_seq_len",
                                         "latent_dim", "rope_dim", "nope_dim", "v_dim", "n_experts", "top_k",
                                         "expert_dim", "n_shared", "rope_theta", "norm_eps")}
        kw["tie_embeddings"] = not c.untied_lm_head
        kw.update(overrides)
        return cls(**kw)


class HipLatModel:
    """Device copy of a latent-attention MoE decoder plus its latent cache slots."""

    def __init__(self, cfg: LatConfig, max_batch=1, max_rows=128, device=0):
        self.cfg = cfg
        c = _LatCfg(cfg.vocab_size, cfg.hidden_dim, cfg.n_layers, cfg.n_heads, cfg.max_seq_len, cfg.rope_theta,
                    cfg.norm_eps, cfg.latent_dim, cfg.rope_dim, cfg.nope_dim, cfg.v_dim, cfg.n_experts, cfg.top_k,
                    cfg.expert_dim, cfg.n_shared, cfg.expert_format, cfg.attn_format, cfg.lm_head_format,
                    cfg.kv_format, max_batch, max_rows, 0 if cfg.tie_embeddings else 1)
        h = _P()
        st = lib().aarh_lat_create(device, C.byref(c), C.byref(h))
        self.h = h
        if st:
            msg = lib().aarh_lat_last_error(h).decode() if h else "aarh_lat_create failed"
            self.close()
            raise _ERRS.get(st, AarambhError)(msg)
        self.max_batch = max_batch
        self.max_rows = max_rows
        _LIVE.add(self)

    def close(self):
        if getattr(self, "h", None):
            lib().aarh_lat_destroy(self.h)
            self.h = None

    def __del__(self):
        self.close()

    def _check(self, st):
        if st:
            raise _ERRS.get(st, AarambhError)(lib().aarh_lat_last_error(self.h).decode())

    def tensors(self):
        out = []
        name = C.create_string_buffer(160)
        for i in range(lib().aarh_lat_num_tensors(self.h)):
            r, c, k = C.c_int64(), C.c_int64(), C.c_int32()
            self._check(lib().aarh_lat_tensor_info(self.h, i, name, 160, C.byref(r), C.byref(c), C.byref(k)))
            out.append((name.value.decode(), r.value, c.value, k.value))
        return out

    def load_f32(self, tid, values):
        v = np.ascontiguousarray(values, np.float32)
        self._check(lib().aarh_lat_load_tensor_f32(self.h, tid, _ptr(v), v.size))

    def load_packed_i4(self, tid, t: PackedInt4Tensor):
        """A PackedInt4Tensor into an INT4 g128 tensor (aarh_lat_load_tensor_packed_i4)."""
        shape, data, sc, zz = t._args()
        self._check(lib().aarh_lat_load_tensor_packed_i4(self.h, tid, _ptr(shape), shape.size, int(t.group_size),
                                                         _ptr(data), data.size, _ptr(sc), _ptr(zz), sc.size))

    def init_synthetic(self, seed=0, std=0.02):
        self._check(lib().aarh_lat_init_synthetic(self.h, seed, std))

    def load_gguf(self, path):
        """Every tensor of an MLA + MoE GGUF v1 checkpoint (aarh_lat_load_gguf); returns the count."""
        n = C.c_int32()
        self._check(lib().aarh_lat_load_gguf(self.h, os.fsencode(path), C.byref(n)))
        return n.value

    def load_safetensors(self, path):
        """Every tensor of an MLA + MoE safetensors checkpoint (aarh_lat_load_safetensors)."""
        n = C.c_int32()
        self._check(lib().aarh_lat_load_safetensors(self.h, os.fsencode(path), C.byref(n)))
        return n.value

    def kv_len(self, slot=0):
        v = C.c_int32()
        self._check(lib().aarh_lat_kv_len(self.h, slot, C.byref(v)))
        return v.value

    def snapshot(self, slot=0):
        return self.kv_len(slot)

    def restore(self, snapshot, slot=0):
        self._check(lib().aarh_lat_kv_rollback(self.h, slot, snapshot))

    def kv_fill_synthetic(self, slot, length, seed=0):
        self._check(lib().aarh_lat_kv_fill_synthetic(self.h, slot, length, seed))

    def forward_with_cache_output(self, ids, offsets, slots=None, want_logits=True, want_hidden=True):
        """ids [nseq, S]; returns (logits [nseq, S, V], hidden [nseq, S, H])."""
        ids = np.ascontiguousarray(np.atleast_2d(ids), np.uint32)
        nseq, S = ids.shape
        offs = np.ascontiguousarray(np.broadcast_to(np.asarray(offsets, np.int32), (nseq,)), np.int32)
        sl = np.ascontiguousarray(np.arange(nseq, dtype=np.int32) if slots is None else slots, np.int32)
        lg = np.empty((nseq, S, self.cfg.vocab_size), np.float32) if want_logits else None
        hd = np.empty((nseq, S, self.cfg.hidden_dim), np.float32) if want_hidden else None
        self._check(lib().aarh_lat_forward(self.h, _ptr(ids), _ptr(sl), _ptr(offs), nseq, S, _ptr(lg), _ptr(hd)))
        self._last_rows = nseq * S
        return lg, hd

    def router_gaps(self):
        """Smallest k-th minus (k+1)-th router logit per row of the last forward, over all layers."""
        out = np.empty(getattr(self, "_last_rows", 0), np.float32)
        self._check(lib().aarh_lat_router_gaps(self.h, _ptr(out)))
        return out

    def expert_counts(self):
        """Rows routed to each expert per layer in the last forward, [n_layers, n_experts + n_shared]."""
        out = np.empty((self.cfg.n_layers, self.cfg.n_experts + self.cfg.n_shared), np.int32)
        self._check(lib().aarh_lat_expert_counts(self.h, _ptr(out)))
        return out

    def prof_enable(self, on=True):
        self._check(lib().aarh_lat_prof_enable(self.h, 1 if on else 0))

    def prof_get(self):
        out = {}
        for i, n in enumerate(PROF_NAMES):
            ms, by, cnt = C.c_double(), C.c_double(), C.c_int64()
            self._check(lib().aarh_lat_prof_get(self.h, i, C.byref(ms), C.byref(by), C.byref(cnt)))
            out[n] = {"ms": ms.value, "bytes": by.value, "launches": cnt.value}
        return out
