"""ctypes bindings for the CPU oracle (oracle/librefcpu.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, never by the product library.
"""
import ctypes as C
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "librefcpu.so")

REF_OK, REF_ERR_CONFIG, REF_ERR_SHAPE, REF_ERR_UNSUPPORTED = 0, 1, 2, 3
W_F32, W_BF16, W_INT8_ROW, W_INT4_G128 = 0, 1, 2, 3
KV_F32, KV_F16, KV_INT8 = 0, 1, 2
T_NORM, T_LINEAR, T_EMBED = 0, 1, 2
FLAG_RATIO_NEAR, FLAG_CDF_NEAR, FLAG_ARGMAX_NEAR, FLAG_TOPP_NEAR = 1, 2, 4, 8
FINISH_MAX_TOKENS, FINISH_EOS, FINISH_CONTEXT_LIMIT = 0, 1, 2


class RefRng(C.Structure):
    _fields_ = [("key", C.c_uint32 * 8), ("pos", C.c_uint64), ("cached_block", C.c_uint64),
                ("buf", C.c_uint32 * 16)]


class RefSampler(C.Structure):
    _fields_ = [("greedy", C.c_int32), ("temperature", C.c_float), ("top_k", C.c_int32),
                ("top_p", C.c_float)]


class RefAcceptResult(C.Structure):
    _fields_ = [("accept_len", C.c_int32), ("token", C.c_int32), ("flags", C.c_uint32),
                ("draws", C.c_int32), ("ratio_margin", C.c_float), ("cdf_margin", C.c_float)]


class RefRound(C.Structure):
    """One engine round: start state (committed tokens, keystream position), outcome and
    the smallest distance of any of its decisions to the boundary that would flip it."""
    _fields_ = [("rng_pos_before", C.c_uint64), ("rng_pos_after", C.c_uint64),
                ("committed_before", C.c_int32), ("committed_after", C.c_int32),
                ("proposed", C.c_int32), ("accepted", C.c_int32),
                ("prob_margin", C.c_float), ("logit_gap", C.c_float)]

    def as_dict(self):
        return {n: getattr(self, n) for n, _ in self._fields_}


class RefConfig(C.Structure):
    _fields_ = [(n, C.c_int32) for n in ("vocab_size", "hidden_dim", "ffn_dim", "n_layers",
                                          "n_heads", "n_kv_heads", "max_seq_len")] + \
               [("rope_theta", C.c_float), ("norm_eps", C.c_float)] + \
               [(n, C.c_int32) for n in ("num_future_tokens", "weight_format",
                                          "lm_head_format", "kv_format", "untied_lm_head")]


class RefLatConfig(C.Structure):
    _fields_ = [(n, C.c_int32) for n in ("vocab_size", "hidden_dim", "n_layers", "n_heads", "max_seq_len")] + \
               [("rope_theta", C.c_float), ("norm_eps", C.c_float)] + \
               [(n, C.c_int32) for n in ("latent_dim", "rope_dim", "nope_dim", "v_dim", "n_experts", "top_k",
                                          "expert_dim", "n_shared", "expert_format", "attn_format",
                                          "lm_head_format", "kv_format", "untied_lm_head")]


class RefSpecStats(C.Structure):
    _fields_ = [(n, C.c_int32) for n in ("rounds", "draft_tokens_proposed", "draft_tokens_accepted",
                                          "draft_tokens_rejected", "target_decode_forwards",
                                          "draft_decode_forwards", "mtp_head_forwards")]

    def as_dict(self):
        return {n: getattr(self, n) for n, _ in self._fields_}


_lib = None

F32P = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")
U32P = np.ctypeslib.ndpointer(np.uint32, flags="C_CONTIGUOUS")
U16P = np.ctypeslib.ndpointer(np.uint16, flags="C_CONTIGUOUS")
U8P = np.ctypeslib.ndpointer(np.uint8, flags="C_CONTIGUOUS")
I8P = np.ctypeslib.ndpointer(np.int8, flags="C_CONTIGUOUS")
I32P = np.ctypeslib.ndpointer(np.int32, flags="C_CONTIGUOUS")
U64P = np.ctypeslib.ndpointer(np.uint64, flags="C_CONTIGUOUS")


def lib():
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(f"oracle library missing: {LIB_PATH} (run __graft_entry__.build())")
    L = C.CDLL(LIB_PATH)
    sig = {
        "ref_chacha_core": (None, [np.ctypeslib.ndpointer(np.uint32), C.c_int, np.ctypeslib.ndpointer(np.uint32)]),
        "ref_pcg32_xsh_rr": (C.c_uint32, [C.c_uint64]),
        "ref_rng_seed_u64": (None, [C.POINTER(RefRng), C.c_uint64]),
        "ref_rng_set_pos": (None, [C.POINTER(RefRng), C.c_uint64]),
        "ref_rng_next_u32": (C.c_uint32, [C.POINTER(RefRng)]),
        "ref_rng_next_f32": (C.c_float, [C.POINTER(RefRng)]),
        "ref_rng_word_f32": (C.c_float, [C.c_uint64, C.c_uint64]),
        "ref_is_deterministic": (C.c_int, [C.POINTER(RefSampler)]),
        "ref_argmax": (C.c_int64, [F32P, C.c_int64]),
        "ref_probabilities": (C.c_int, [C.POINTER(RefSampler), F32P, C.c_int64, F32P]),
        "ref_validate_probabilities": (C.c_int, [F32P, C.c_int64]),
        "ref_sample_probabilities": (C.c_int, [C.POINTER(RefSampler), C.POINTER(RefRng), F32P, C.c_int64,
                                               C.POINTER(C.c_uint32), C.POINTER(C.c_float), C.POINTER(C.c_float)]),
        "ref_accept_proposal": (C.c_int, [C.POINTER(RefSampler), C.POINTER(RefRng), C.c_uint32, F32P, F32P,
                                          C.c_int64, C.POINTER(C.c_int), C.POINTER(C.c_float),
                                          C.POINTER(C.c_float), C.POINTER(C.c_int)]),
        "ref_residual": (C.c_int, [F32P, F32P, C.c_int64, F32P]),
        "ref_accept_batch": (C.c_int, [C.c_int, C.c_int, C.c_int64, F32P, C.c_int, F32P, U32P, C.c_void_p,
                                       C.c_int, C.POINTER(RefSampler), C.c_void_p, C.c_void_p, C.c_void_p,
                                       C.POINTER(RefAcceptResult)]),
        "ref_f32_to_f16": (C.c_uint16, [C.c_float]),
        "ref_f16_to_f32": (C.c_float, [C.c_uint16]),
        "ref_f32_to_bf16": (C.c_uint16, [C.c_float]),
        "ref_bf16_to_f32": (C.c_float, [C.c_uint16]),
        "ref_quantise_i4": (C.c_int, [F32P, C.c_int64, C.c_int64, U8P, F32P, F32P]),
        "ref_dequantise_i4": (C.c_int, [U8P, C.c_int64, C.c_int64, F32P, F32P, F32P]),
        "ref_quantise_i4_f16": (C.c_int, [F32P, C.c_int64, C.c_int64, U8P, U16P, U16P]),
        "ref_dequantise_i4_f16": (C.c_int, [U8P, C.c_int64, C.c_int64, U16P, U16P, F32P]),
        "ref_quantise_i8_rows": (C.c_int, [F32P, C.c_int64, C.c_int64, I8P, F32P]),
        "ref_quantise_kv_row": (C.c_int, [F32P, C.c_int64, I8P, U16P]),
        "ref_splitmix64": (C.c_uint64, [C.c_uint64]),
        "ref_synth_normal": (C.c_float, [C.c_uint64, C.c_uint32, C.c_uint64]),
        "ref_synth_fill": (None, [C.c_uint64, C.c_uint32, C.c_int64, C.c_float, F32P]),
        "ref_synth_tokens": (None, [C.c_uint64, C.c_uint32, C.c_int64, C.c_uint32, U32P]),
        "ref_model_create": (C.c_void_p, [C.POINTER(RefConfig)]),
        "ref_rope_frequencies": (C.c_int, [C.c_int, C.c_double, C.c_int, C.c_int, C.c_double, C.c_int,
                                           C.c_double, C.c_double, C.c_double, F32P, C.POINTER(C.c_float),
                                           C.c_char_p, C.c_int]),
        "ref_model_set_rope_scaling": (C.c_int, [C.c_void_p, C.c_int, C.c_double, C.c_int, C.c_double,
                                                 C.c_double, C.c_double, C.c_char_p, C.c_int]),
        "ref_model_free": (None, [C.c_void_p]),
        "ref_model_num_tensors": (C.c_int, [C.c_void_p]),
        "ref_model_tensor_info": (C.c_int, [C.c_void_p, C.c_int, C.c_char_p, C.c_int, C.POINTER(C.c_int64),
                                            C.POINTER(C.c_int64), C.POINTER(C.c_int32)]),
        "ref_model_set_tensor": (C.c_int, [C.c_void_p, C.c_int, F32P]),
        "ref_model_get_tensor": (C.c_int, [C.c_void_p, C.c_int, F32P]),
        "ref_model_init_synthetic": (C.c_int, [C.c_void_p, C.c_uint64, C.c_float]),
        "ref_kv_create": (C.c_void_p, [C.c_void_p, C.c_int]),
        "ref_kv_free": (None, [C.c_void_p]),
        "ref_kv_len": (C.c_int, [C.c_void_p]),
        "ref_kv_truncate": (C.c_int, [C.c_void_p, C.c_int]),
        "ref_kv_fill_synthetic": (C.c_int, [C.c_void_p, C.c_uint64, C.c_int]),
        "ref_forward": (C.c_int, [C.c_void_p, C.c_void_p, U32P, C.c_int, C.c_int, C.c_void_p, C.c_void_p, C.c_int]),
        "ref_forward_layers": (C.c_int, [C.c_void_p, C.c_void_p, U32P, C.c_int, C.c_int, C.c_int, C.c_int,
                                         C.c_void_p, C.c_int]),
        "ref_mtp_head": (C.c_int, [C.c_void_p, C.c_int, F32P, U32P, C.c_int, F32P, C.c_int]),
        "ref_mtp_generate": (C.c_int, [C.c_void_p, U32P, C.c_int, C.c_int, C.c_int, C.POINTER(RefSampler),
                                       C.c_uint64, C.c_int, U32P, C.POINTER(C.c_int), C.POINTER(C.c_int),
                                       C.POINTER(RefSpecStats), C.POINTER(C.c_float)]),
        "ref_spec_generate": (C.c_int, [C.c_void_p, C.c_void_p, U32P, C.c_int, C.c_int, C.c_int,
                                        C.POINTER(RefSampler), C.c_uint64, C.c_int, U32P, C.POINTER(C.c_int),
                                        C.POINTER(C.c_int), C.POINTER(RefSpecStats), C.POINTER(C.c_float)]),
        "ref_top_candidates": (None, [F32P, C.c_int64, C.c_int, U32P, F32P]),
        "ref_set_candidate_sink": (None, [C.c_void_p, C.c_void_p, C.c_int]),
        "ref_set_round_sink": (None, [C.c_void_p, C.c_int, C.c_void_p]),
        "ref_last_topp_margin": (C.c_float, []),
        "ref_last_topk_gap": (C.c_float, []),
        "ref_lat_create": (C.c_void_p, [C.POINTER(RefLatConfig)]),
        "ref_lat_free": (None, [C.c_void_p]),
        "ref_lat_num_tensors": (C.c_int, [C.c_void_p]),
        "ref_lat_tensor_info": (C.c_int, [C.c_void_p, C.c_int, C.c_char_p, C.c_int, C.POINTER(C.c_int64),
                                          C.POINTER(C.c_int64), C.POINTER(C.c_int32)]),
        "ref_lat_set_tensor": (C.c_int, [C.c_void_p, C.c_int, F32P]),
        "ref_lat_get_tensor": (C.c_int, [C.c_void_p, C.c_int, F32P]),
        "ref_lat_init_synthetic": (C.c_int, [C.c_void_p, C.c_uint64, C.c_float]),
        "ref_lat_kv_create": (C.c_void_p, [C.c_void_p, C.c_int]),
        "ref_lat_kv_free": (None, [C.c_void_p]),
        "ref_lat_kv_truncate": (C.c_int, [C.c_void_p, C.c_int]),
        "ref_lat_kv_fill_synthetic": (C.c_int, [C.c_void_p, C.c_uint64, C.c_int]),
        "ref_lat_forward": (C.c_int, [C.c_void_p, C.c_void_p, U32P, C.c_int, C.c_int, C.c_void_p, C.c_void_p,
                                      C.c_int]),
        "ref_topk_gating": (None, [F32P, C.c_int, C.c_int, C.c_int, I32P, F32P]),
        "ref_plain_generate": (C.c_int, [C.c_void_p, U32P, C.c_int, C.c_int, C.POINTER(RefSampler), C.c_uint64,
                                         C.c_int, U32P, C.POINTER(C.c_int), C.POINTER(C.c_int)]),
    }
    for name, (res, args) in sig.items():
        f = getattr(L, name)
        f.restype = res
        f.argtypes = args
    _lib = L
    return L


def _ptr(a):
    return None if a is None else a.ctypes.data_as(C.c_void_p)


def sampler(greedy=False, temperature=1.0, top_k=0, top_p=0.0):
    return RefSampler(1 if greedy else 0, temperature, top_k, top_p)


class Rng:
    """rand 0.8 StdRng (ChaCha12) seeded with seed_from_u64."""

    def __init__(self, seed, pos=0):
        self.s = RefRng()
        lib().ref_rng_seed_u64(C.byref(self.s), seed)
        lib().ref_rng_set_pos(C.byref(self.s), pos)

    def next_u32(self):
        return lib().ref_rng_next_u32(C.byref(self.s))

    def next_f32(self):
        return lib().ref_rng_next_f32(C.byref(self.s))

    @property
    def pos(self):
        return self.s.pos


def chacha_core(state16, rounds):
    inp = np.ascontiguousarray(state16, dtype=np.uint32)
    out = np.zeros(16, np.uint32)
    lib().ref_chacha_core(inp, rounds, out)
    return out


def argmax(v):
    return int(lib().ref_argmax(np.ascontiguousarray(v, np.float32), len(v)))


def probabilities(s, logits, margins=False):
    """Sampler::probabilities (sampler.rs:102-118); with margins=True also returns the
    top-p cumulative margin and the top-k boundary logit gap of the filter."""
    logits = np.ascontiguousarray(logits, np.float32)
    out = np.zeros_like(logits)
    st = lib().ref_probabilities(C.byref(s), logits, len(logits), out)
    if st:
        raise ValueError(f"probabilities failed: status {st}")
    if margins:
        return out, float(lib().ref_last_topp_margin()), float(lib().ref_last_topk_gap())
    return out


def residual(target, draft):
    target = np.ascontiguousarray(target, np.float32)
    draft = np.ascontiguousarray(draft, np.float32)
    out = np.zeros_like(target)
    st = lib().ref_residual(target, draft, len(target), out)
    if st:
        raise ValueError(f"residual failed: status {st}")
    return out


def sample_probabilities(s, rng, p):
    p = np.ascontiguousarray(p, np.float32)
    tok = C.c_uint32()
    st = lib().ref_sample_probabilities(C.byref(s), C.byref(rng.s), p, len(p), C.byref(tok), None, None)
    if st:
        raise ValueError(f"sample failed: status {st}")
    return int(tok.value)


def accept_proposal(s, rng, token, draft, target):
    draft = np.ascontiguousarray(draft, np.float32)
    target = np.ascontiguousarray(target, np.float32)
    acc, drew = C.c_int(), C.c_int()
    lib().ref_accept_proposal(C.byref(s), C.byref(rng.s), token, draft, target, len(draft),
                              C.byref(acc), None, None, C.byref(drew))
    return bool(acc.value)


def accept_batch(target, draft, draft_tokens, s, bonus, seeds=None, word_offsets=None,
                 uniforms=None, n_proposals=None):
    """target [B, Kt, V], draft [B, K, V], draft_tokens [B, K]."""
    target = np.ascontiguousarray(target, np.float32)
    draft = np.ascontiguousarray(draft, np.float32)
    toks = np.ascontiguousarray(draft_tokens, np.uint32)
    B, K, V = draft.shape
    res = (RefAcceptResult * B)()
    keep = []

    def opt(a, dt):
        if a is None:
            return None
        a = np.ascontiguousarray(a, dt)
        keep.append(a)
        return _ptr(a)

    st = lib().ref_accept_batch(B, K, V, target, target.shape[1], draft, toks,
                                opt(n_proposals, np.int32), 1 if bonus else 0, C.byref(s),
                                opt(seeds, np.uint64), opt(word_offsets, np.uint64),
                                opt(uniforms, np.float32), res)
    if st:
        raise ValueError(f"accept_batch failed: status {st}")
    return {
        "accept_len": np.array([r.accept_len for r in res], np.int32),
        "token": np.array([r.token for r in res], np.int32),
        "flags": np.array([r.flags for r in res], np.uint32),
        "draws": np.array([r.draws for r in res], np.int32),
        "ratio_margin": np.array([r.ratio_margin for r in res], np.float32),
        "cdf_margin": np.array([r.cdf_margin for r in res], np.float32),
    }


def f32_to_f16_bits(x):
    return np.array([lib().ref_f32_to_f16(float(v)) for v in np.ravel(x)], np.uint16)


def quantise_i4(w, group):
    w = np.ascontiguousarray(w, np.float32).ravel()
    n = w.size
    ng = -(-n // group)
    packed = np.zeros((n + 1) // 2, np.uint8)
    sc = np.zeros(ng, np.float32)
    zz = np.zeros(ng, np.float32)
    lib().ref_quantise_i4(w, n, group, packed, sc, zz)
    return packed, sc, zz


def dequantise_i4(packed, n, group, sc, zz):
    out = np.zeros(n, np.float32)
    lib().ref_dequantise_i4(np.ascontiguousarray(packed, np.uint8), n, group,
                            np.ascontiguousarray(sc, np.float32), np.ascontiguousarray(zz, np.float32), out)
    return out


def quantise_i4_f16(w, group=128):
    w = np.ascontiguousarray(w, np.float32).ravel()
    n = w.size
    ng = -(-n // group)
    packed = np.zeros((n + 1) // 2, np.uint8)
    sh = np.zeros(ng, np.uint16)
    zh = np.zeros(ng, np.uint16)
    lib().ref_quantise_i4_f16(w, n, group, packed, sh, zh)
    return packed, sh, zh


def dequantise_i4_f16(packed, n, group, sh, zh):
    out = np.zeros(n, np.float32)
    lib().ref_dequantise_i4_f16(np.ascontiguousarray(packed, np.uint8), n, group,
                                np.ascontiguousarray(sh, np.uint16), np.ascontiguousarray(zh, np.uint16), out)
    return out


def quantise_i8_rows(w):
    w = np.ascontiguousarray(w, np.float32)
    rows, cols = w.shape
    codes = np.zeros((rows, cols), np.int8)
    sc = np.zeros(rows, np.float32)
    lib().ref_quantise_i8_rows(w, rows, cols, codes, sc)
    return codes, sc


def quantise_kv_row(x):
    x = np.ascontiguousarray(x, np.float32)
    codes = np.zeros(x.size, np.int8)
    sh = np.zeros(1, np.uint16)
    lib().ref_quantise_kv_row(x, x.size, codes, sh)
    return codes, int(sh[0])


TOP_CANDIDATES = 5  # engine.rs:70


def top_candidates(p, k=TOP_CANDIDATES):
    """Sampler::top_candidates_from_probabilities (sampler.rs:188-208): (ids, probs)."""
    p = np.ascontiguousarray(p, np.float32)
    ids = np.zeros(k, np.uint32)
    probs = np.zeros(k, np.float32)
    lib().ref_top_candidates(p, p.size, k, ids, probs)
    return ids, probs


def synth_fill(seed, stream, n, std):
    out = np.zeros(n, np.float32)
    lib().ref_synth_fill(seed, stream, n, std, out)
    return out


def synth_tokens(seed, stream, n, vocab):
    out = np.zeros(n, np.uint32)
    lib().ref_synth_tokens(seed, stream, n, vocab, out)
    return out


def make_config(vocab_size, hidden_dim, ffn_dim, n_layers, n_heads, n_kv_heads, max_seq_len,
                rope_theta=10000.0, norm_eps=1e-5, num_future_tokens=0, weight_format=W_F32,
                lm_head_format=0, kv_format=KV_F32, untied_lm_head=0):
    return RefConfig(vocab_size, hidden_dim, ffn_dim, n_layers, n_heads, n_kv_heads, max_seq_len,
                     rope_theta, norm_eps, num_future_tokens, weight_format, lm_head_format, kv_format,
                     int(untied_lm_head))


ROPE_METHODS = {None: 0, "none": 0, "yarn": 1, "ntk": 2, "linear": 3}


def _rope_args(scaling):
    """(method, factor, original_max_seq_len, beta_fast, beta_slow, attn_factor) of a mapping
    with RopeScalingConfig's fields (config.rs:22-47 defaults: yarn, 32, 1, attn 1)."""
    if scaling is None:
        return (0, 0.0, 0, 0.0, 0.0, 0.0)
    g = scaling.get if isinstance(scaling, dict) else (lambda k, d=None: getattr(scaling, k, d))
    return (ROPE_METHODS[g("method", "yarn")], float(g("factor", 1.0)), int(g("original_max_seq_len", 0)),
            float(g("beta_fast", 32.0)), float(g("beta_slow", 1.0)), float(g("attn_factor", 1.0)))


def rope_frequencies(head_dim, theta, max_seq_len, scaling=None):
    """inverse_frequencies_for_config (rope_scaling.rs:24-33): (inv_freq f32[hd/2], attn_factor);
    ValueError with RopeScalingConfig::validate's message on a bad config."""
    inv = np.zeros(max(head_dim // 2, 1), np.float32)
    attn = C.c_float()
    err = C.create_string_buffer(256)
    r = lib().ref_rope_frequencies(head_dim, theta, max_seq_len, *_rope_args(scaling), inv, C.byref(attn), err, 256)
    if r:
        raise ValueError(err.value.decode())
    return inv[: head_dim // 2], attn.value


class Model:
    def __init__(self, cfg, seed=None, std=0.02):
        self.cfg = cfg
        self.h = lib().ref_model_create(C.byref(cfg))
        if not self.h:
            raise ValueError("invalid oracle model config")
        if seed is not None:
            st = lib().ref_model_init_synthetic(self.h, seed, std)
            if st:
                raise ValueError(f"synthetic init failed: {st}")

    def set_rope_scaling(self, scaling):
        """RopeCache::from_config with cfg.rope_scaling = scaling (None: unscaled)."""
        err = C.create_string_buffer(256)
        if lib().ref_model_set_rope_scaling(self.h, *_rope_args(scaling), err, 256):
            raise ValueError(err.value.decode())

    def close(self):
        if self.h:
            lib().ref_model_free(self.h)
            self.h = None

    def __del__(self):
        self.close()

    def tensors(self):
        out = []
        name = C.create_string_buffer(128)
        for i in range(lib().ref_model_num_tensors(self.h)):
            r, c, k = C.c_int64(), C.c_int64(), C.c_int32()
            lib().ref_model_tensor_info(self.h, i, name, 128, C.byref(r), C.byref(c), C.byref(k))
            out.append((name.value.decode(), r.value, c.value, k.value))
        return out

    def get(self, i):
        _, r, c, _ = self.tensors()[i]
        out = np.zeros(r * c, np.float32)
        lib().ref_model_get_tensor(self.h, i, out)
        return out.reshape(r, c)

    def set(self, i, raw):
        st = lib().ref_model_set_tensor(self.h, i, np.ascontiguousarray(raw, np.float32).ravel())
        if st:
            raise ValueError(f"set_tensor failed: {st}")

    def kv(self, capacity):
        return KvCache(self, capacity)

    def mtp_head(self, head, anchor, ids, nthreads=8):
        out = np.zeros(self.cfg.vocab_size, np.float32)
        ids = np.ascontiguousarray(ids, np.uint32)
        st = lib().ref_mtp_head(self.h, head, np.ascontiguousarray(anchor, np.float32), ids, len(ids), out, nthreads)
        if st:
            raise ValueError(f"mtp_head failed: {st}")
        return out

    def _sink(self, max_new):
        """Record the top-5 candidates of every committed token of the next engine call
        (Sampler::top_candidates_from_probabilities) in self.last_candidates."""
        ids = np.zeros((max(max_new, 1), TOP_CANDIDATES), np.uint32)
        probs = np.zeros((max(max_new, 1), TOP_CANDIDATES), np.float32)
        lib().ref_set_candidate_sink(_ptr(ids), _ptr(probs), max(max_new, 1))
        return ids, probs

    def _unsink(self, ids, probs, n):
        lib().ref_set_candidate_sink(None, None, 0)
        self.last_candidates = (ids[:n].copy(), probs[:n].copy())

    def _round_sink(self, max_new):
        """Record the rounds of the next engine call in self.last_rounds (list of dicts)."""
        buf = (RefRound * (max(max_new, 1) + 2))()
        cnt = C.c_int(0)
        lib().ref_set_round_sink(C.cast(buf, C.c_void_p), len(buf), C.addressof(cnt))
        return buf, cnt

    def _round_unsink(self, buf, cnt):
        lib().ref_set_round_sink(None, 0, None)
        self.last_rounds = [buf[i].as_dict() for i in range(min(cnt.value, len(buf)))]

    def mtp_generate(self, prompt, max_new, num_draft, s, seed=0, nthreads=8):
        prompt = np.ascontiguousarray(prompt, np.uint32)
        out = np.zeros(max(max_new, 1), np.uint32)
        n, fin, gap = C.c_int(), C.c_int(), C.c_float()
        stats = RefSpecStats()
        ci, cp = self._sink(max_new)
        rb, rc = self._round_sink(max_new)
        st = lib().ref_mtp_generate(self.h, prompt, len(prompt), max_new, num_draft, C.byref(s), seed,
                                    nthreads, out, C.byref(n), C.byref(fin), C.byref(stats), C.byref(gap))
        self._unsink(ci, cp, n.value)
        self._round_unsink(rb, rc)
        if st:
            raise ValueError(f"mtp_generate failed: {st}")
        return out[:n.value].copy(), fin.value, stats.as_dict(), gap.value

    def spec_generate(self, draft, prompt, max_new, num_draft, s, seed=0, nthreads=8):
        """SpeculativeEngine::generate_with_callback (speculative.rs:175-516) with `draft`
        (another Model) as the external draft model."""
        prompt = np.ascontiguousarray(prompt, np.uint32)
        out = np.zeros(max(max_new, 1), np.uint32)
        n, fin, gap = C.c_int(), C.c_int(), C.c_float()
        stats = RefSpecStats()
        ci, cp = self._sink(max_new)
        rb, rc = self._round_sink(max_new)
        st = lib().ref_spec_generate(self.h, draft.h, prompt, len(prompt), max_new, num_draft, C.byref(s), seed,
                                     nthreads, out, C.byref(n), C.byref(fin), C.byref(stats), C.byref(gap))
        self._unsink(ci, cp, n.value)
        self._round_unsink(rb, rc)
        if st:
            raise ValueError(f"spec_generate failed: {st}")
        return out[:n.value].copy(), fin.value, stats.as_dict(), gap.value

    def plain_generate(self, prompt, max_new, s, seed=0, nthreads=8):
        prompt = np.ascontiguousarray(prompt, np.uint32)
        out = np.zeros(max(max_new, 1), np.uint32)
        n, fin = C.c_int(), C.c_int()
        st = lib().ref_plain_generate(self.h, prompt, len(prompt), max_new, C.byref(s), seed, nthreads, out,
                                      C.byref(n), C.byref(fin))
        if st:
            raise ValueError(f"plain_generate failed: {st}")
        return out[:n.value].copy(), fin.value


class KvCache:
    def __init__(self, model, capacity):
        self.model = model
        self.h = lib().ref_kv_create(model.h, capacity)
        if not self.h:
            raise MemoryError("oracle kv allocation failed")

    def close(self):
        if self.h:
            lib().ref_kv_free(self.h)
            self.h = None

    def __del__(self):
        self.close()

    def __len__(self):
        return lib().ref_kv_len(self.h)

    def truncate(self, n):
        st = lib().ref_kv_truncate(self.h, n)
        if st:
            raise ValueError(f"truncate failed: {st}")

    def fill_synthetic(self, seed, length):
        st = lib().ref_kv_fill_synthetic(self.h, seed, length)
        if st:
            raise ValueError(f"fill failed: {st}")

    def forward(self, ids, offset, want_hidden=True, nthreads=8):
        cfg = self.model.cfg
        ids = np.ascontiguousarray(ids, np.uint32)
        S = len(ids)
        logits = np.zeros((S, cfg.vocab_size), np.float32)
        hidden = np.zeros((S, cfg.hidden_dim), np.float32) if want_hidden else None
        st = lib().ref_forward(self.model.h, self.h, ids, S, offset, _ptr(logits), _ptr(hidden), nthreads)
        if st:
            raise ValueError(f"forward failed: status {st}")
        return logits, hidden

    def forward_layers(self, ids, offset, n_layers, with_head=True, nthreads=8):
        cfg = self.model.cfg
        ids = np.ascontiguousarray(ids, np.uint32)
        S = len(ids)
        logits = np.zeros((S, cfg.vocab_size), np.float32) if with_head else None
        st = lib().ref_forward_layers(self.model.h, self.h, ids, S, offset, n_layers, 1 if with_head else 0,
                                      _ptr(logits), nthreads)
        if st:
            raise ValueError(f"forward_layers failed: status {st}")
        return logits


# ---------------- latent-attention MoE decoder (benchmark config 5) ----------------
def make_lat_config(vocab_size, hidden_dim, n_layers, n_heads, max_seq_len, latent_dim, rope_dim, nope_dim, v_dim,
                    n_experts, top_k, expert_dim, n_shared, expert_format=W_F32, attn_format=W_F32,
                    lm_head_format=0, kv_format=KV_F32, rope_theta=10000.0, norm_eps=1e-5, untied_lm_head=0):
    return RefLatConfig(vocab_size, hidden_dim, n_layers, n_heads, max_seq_len, rope_theta, norm_eps, latent_dim,
                        rope_dim, nope_dim, v_dim, n_experts, top_k, expert_dim, n_shared, expert_format,
                        attn_format, lm_head_format, kv_format, untied_lm_head)


def topk_gating(logits, k):
    """top_k_gating (moe.rs:361-406): selected expert indices and softmax weights per row."""
    logits = np.ascontiguousarray(np.atleast_2d(logits), np.float32)
    rows, E = logits.shape
    idx = np.zeros((rows, k), np.int32)
    w = np.zeros((rows, k), np.float32)
    lib().ref_topk_gating(logits, rows, E, k, idx, w)
    return idx, w


class LatModel:
    """MLA + MoE decoder oracle (mla.rs:300-489, moe.rs:212-406), f32 compute on the
    effective (dequantised) weights."""

    def __init__(self, cfg):
        self.cfg = cfg
        self.h = lib().ref_lat_create(C.byref(cfg))
        if not self.h:
            raise ValueError("invalid latent MoE config")

    def close(self):
        if self.h:
            lib().ref_lat_free(self.h)
            self.h = None

    def __del__(self):
        self.close()

    def tensors(self):
        out = []
        for i in range(lib().ref_lat_num_tensors(self.h)):
            name = C.create_string_buffer(128)
            r, c, k = C.c_int64(), C.c_int64(), C.c_int32()
            lib().ref_lat_tensor_info(self.h, i, name, 128, C.byref(r), C.byref(c), C.byref(k))
            out.append((name.value.decode(), r.value, c.value, k.value))
        return out

    def get(self, i):
        name, r, c, k = self.tensors()[i]
        out = np.zeros(r * c, np.float32)
        lib().ref_lat_get_tensor(self.h, i, out)
        return out.reshape(r, c)

    def set(self, i, raw):
        st = lib().ref_lat_set_tensor(self.h, i, np.ascontiguousarray(raw, np.float32).ravel())
        if st:
            raise ValueError(f"set_tensor {i} failed: {st}")

    def init_synthetic(self, seed, std):
        """Random-init weights on the streams the device's synthetic init uses
        (router ~ N(0, 1/hidden) for unit-variance logits)."""
        st = lib().ref_lat_init_synthetic(self.h, seed, std)
        if st:
            raise ValueError(f"synthetic init failed: {st}")

    def kv(self, capacity):
        return LatKv(self, capacity)


class LatKv:
    def __init__(self, model, capacity):
        self.model = model
        self.h = lib().ref_lat_kv_create(model.h, capacity)
        if not self.h:
            raise MemoryError("oracle latent cache allocation failed")

    def close(self):
        if self.h:
            lib().ref_lat_kv_free(self.h)
            self.h = None

    def __del__(self):
        self.close()

    def truncate(self, n):
        st = lib().ref_lat_kv_truncate(self.h, n)
        if st:
            raise ValueError(f"truncate failed: {st}")

    def fill_synthetic(self, seed, length):
        st = lib().ref_lat_kv_fill_synthetic(self.h, seed, length)
        if st:
            raise ValueError(f"fill failed: {st}")

    def forward(self, ids, offset, want_hidden=True, nthreads=8):
        cfg = self.model.cfg
        ids = np.ascontiguousarray(ids, np.uint32)
        S = len(ids)
        logits = np.zeros((S, cfg.vocab_size), np.float32)
        hidden = np.zeros((S, cfg.hidden_dim), np.float32) if want_hidden else None
        st = lib().ref_lat_forward(self.model.h, self.h, ids, S, offset, _ptr(logits), _ptr(hidden), nthreads)
        if st:
            raise ValueError(f"forward failed: status {st}")
        return logits, hidden
