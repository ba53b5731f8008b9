"""Checkpoint containers of aarambh-studio restated in numpy -- TEST INFRASTRUCTURE ONLY.

Nothing on the product path imports this module: the tests use it to write
fixtures and to decode them the way the reference does, as the checker of the
library's own readers (aarh_load_gguf, aarh_load_safetensors, aarh_gguf_read_tensor).

  GGUF v1 container      weights/src/gguf.rs:47-134 (save_gguf, load_gguf_tensors)
  tensor encodings       gguf.rs:127-241 (F32, Q8_0 per-tensor absmax, Q4_K_M blocks)
  Q4_K_M block codec     quant/src/gguf_quant.rs:1-49
  f32 <-> f16 (custom)   quant/src/gguf_quant.rs:51-112 (round half up on the mantissa)
  absmax INT8            quant/src/absmax.rs:7-24, dequant.rs:7-16
  safetensors            weights/src/lib.rs:68-99 (save_model / load_model via candle)
"""
import json
import struct

import numpy as np

MAGIC = b"GGUF"
VERSION = 1
ENC_F32, ENC_Q8_0, ENC_Q4KM = 0, 1, 2  # TensorEncoding, gguf.rs:24-29
Q4KM_BLOCK = 256                        # gguf_quant.rs:2
Q4KM_BYTES = 132                        # gguf_quant.rs:4
F32_EPS = np.float32(np.finfo(np.float32).eps)


def rust_round(x):
    """f32::round: half away from zero, evaluated exactly (x is f32, so float64 holds it)."""
    xd = np.asarray(x, np.float64)
    t = np.trunc(xd)
    return np.where(np.abs(xd - t) >= 0.5, t + np.sign(xd), t)


def f32_to_f16(values):
    """gguf_quant.rs:52-83: truncate the mantissa, add one ulp when the first dropped bit
    is set (round half up in magnitude); overflow to inf, underflow to signed zero."""
    bits = np.asarray(values, np.float32).reshape(-1).view(np.uint32).astype(np.int64)
    sign = (bits >> 16) & 0x8000
    exp = (bits >> 23) & 0xFF
    mant = bits & 0x7FFFFF
    out = np.zeros(bits.shape, np.int64)
    half_exp = exp - 127 + 15
    # inf / nan
    m = exp == 255
    out[m] = sign[m] | np.where(mant[m] == 0, 0x7C00, 0x7E00)
    # overflow
    m2 = ~m & (half_exp >= 31)
    out[m2] = sign[m2] | 0x7C00
    # subnormal half (or zero)
    m3 = ~m & ~m2 & (half_exp <= 0)
    tiny = m3 & (half_exp < -10)
    out[tiny] = sign[tiny]
    sub = m3 & ~tiny
    if sub.any():
        mm = mant[sub] | 0x800000
        shift = 14 - half_exp[sub]
        hm = mm >> shift
        hm = hm + ((mm >> (shift - 1)) & 1)
        out[sub] = sign[sub] | (hm & 0xFFFF)
    # normal
    nm = ~m & ~m2 & ~m3
    h = sign[nm] | (half_exp[nm] << 10) | (mant[nm] >> 13)
    h = h + ((mant[nm] & 0x1000) != 0)
    out[nm] = h & 0xFFFF
    return out.astype(np.uint16).reshape(np.shape(values))


def f16_to_f32(h):
    """gguf_quant.rs:86-112: IEEE binary16 to binary32 (exact)."""
    return np.asarray(h, np.uint16).view(np.float16).astype(np.float32)


def quantise_block_q4km(block):
    """quantise_block_q4_k_m (gguf_quant.rs:7-34) of 256 f32 values -> 132 bytes."""
    block = np.asarray(block, np.float32)
    assert block.shape == (Q4KM_BLOCK,)
    mn = np.float32(np.nanmin(block)) if not np.all(np.isnan(block)) else np.float32(np.inf)
    mx = np.float32(np.nanmax(block)) if not np.all(np.isnan(block)) else np.float32(-np.inf)
    rng = np.float32(mx - mn)
    scale = np.float32(1.0) if np.abs(rng) <= F32_EPS else np.float32(rng / np.float32(15.0))
    with np.errstate(invalid="ignore", over="ignore"):
        q = rust_round((block - mn) / scale)  # f32 subtraction and division, then round
    q = np.clip(np.nan_to_num(q, nan=0.0), 0, 15).astype(np.uint8)
    out = bytearray(Q4KM_BYTES)
    out[0:2] = struct.pack("<H", int(f32_to_f16(scale)))
    out[2:4] = struct.pack("<H", int(f32_to_f16(mn)))
    out[4:] = (q[0::2] | (q[1::2] << 4)).astype(np.uint8).tobytes()
    return bytes(out)


def dequantise_block_q4km(b):
    """dequantise_block_q4_k_m (gguf_quant.rs:37-49): q * scale + min in f32 (two roundings)."""
    scale = f16_to_f32(np.frombuffer(b[0:2], np.uint16))[0]
    mn = f16_to_f32(np.frombuffer(b[2:4], np.uint16))[0]
    codes = np.frombuffer(b[4:Q4KM_BYTES], np.uint8)
    q = np.empty(Q4KM_BLOCK, np.float32)
    q[0::2] = codes & 0x0F
    q[1::2] = codes >> 4
    return (q * scale).astype(np.float32) + mn


def quantise_absmax_i8(values):
    """absmax.rs:7-24: one scale max|v| / 127 (1.0 if <= EPSILON), codes round(v / scale) in [-127, 127]."""
    v = np.asarray(values, np.float32).reshape(-1)
    a = np.abs(v)
    max_abs = np.float32(np.nanmax(a)) if v.size and not np.all(np.isnan(a)) else np.float32(0.0)
    max_abs = max(max_abs, np.float32(0.0))
    scale = np.float32(1.0) if max_abs <= F32_EPS else np.float32(max_abs / np.float32(127.0))
    with np.errstate(invalid="ignore"):
        q = rust_round(v / scale)
    q = np.clip(np.nan_to_num(q, nan=0.0), -127, 127).astype(np.int8)
    return scale, q


def encoding_for(name, shape, fmt):
    """encode_tensor (gguf.rs:127-141): non-2-D tensors and convolution weights stay F32,
    DSA indexer weights Q8_0, other 2-D weights per the file format."""
    if len(shape) != 2 or "_conv." in name:
        return ENC_F32
    if ".dsa.index_" in name:
        return ENC_Q8_0
    return ENC_Q8_0 if fmt == "Q80" else ENC_Q4KM


def encode_tensor(enc, values):
    v = np.ascontiguousarray(values, np.float32).reshape(-1)
    if enc == ENC_F32:
        return v.astype("<f4").tobytes()
    if enc == ENC_Q8_0:
        scale, q = quantise_absmax_i8(v)
        return struct.pack("<f", float(scale)) + q.tobytes()
    nb = (v.size + Q4KM_BLOCK - 1) // Q4KM_BLOCK
    padded = np.zeros(nb * Q4KM_BLOCK, np.float32)
    padded[: v.size] = v
    return b"".join(quantise_block_q4km(padded[i * Q4KM_BLOCK:(i + 1) * Q4KM_BLOCK]) for i in range(nb))


def decode_tensor(enc, shape, payload):
    """decode_tensor (gguf.rs:143-153) to f32 values of `shape`."""
    n = int(np.prod(shape)) if len(shape) else 1
    if enc == ENC_F32:
        if len(payload) % 4:
            raise ValueError("invalid F32 GGUF payload length")
        return np.frombuffer(payload, "<f4").astype(np.float32).reshape(shape)
    if enc == ENC_Q8_0:
        if len(payload) < 4:
            raise ValueError("invalid Q8_0 payload")
        scale = np.float32(struct.unpack("<f", payload[:4])[0])
        q = np.frombuffer(payload[4:], np.int8).astype(np.float32)
        if q.size != n:
            raise ValueError("Q8_0 payload does not match its shape")
        return (q * scale).astype(np.float32).reshape(shape)
    if enc == ENC_Q4KM:
        if len(payload) % Q4KM_BYTES:
            raise ValueError("invalid Q4_K_M GGUF payload length")
        blocks = [dequantise_block_q4km(payload[i:i + Q4KM_BYTES]) for i in range(0, len(payload), Q4KM_BYTES)]
        vals = np.concatenate(blocks) if blocks else np.zeros(0, np.float32)
        return vals[:n].reshape(shape)
    raise ValueError(f"unknown GGUF tensor encoding {enc}")


def model_config_json(vocab_size, hidden_dim, ffn_dim, n_layers, n_heads, n_kv_heads, max_seq_len,
                      rope_theta=10000.0, norm_eps=1e-5, num_future_tokens=0, tie_embeddings=True,
                      rope_scaling=None):
    """ModelConfig (core/src/config.rs:732-776) as serde_json writes it (optional fields omitted)."""
    cfg = {"vocab_size": vocab_size, "hidden_dim": hidden_dim, "ffn_dim": ffn_dim, "n_layers": n_layers,
           "n_heads": n_heads, "n_kv_heads": n_kv_heads, "max_seq_len": max_seq_len, "rope_theta": rope_theta}
    if rope_scaling is not None:
        cfg["rope_scaling"] = dict(rope_scaling)
    if num_future_tokens:
        cfg["mtp"] = {"num_future_tokens": num_future_tokens, "aux_loss_weight": 0.3}
    cfg["norm_eps"] = norm_eps
    cfg["tie_embeddings"] = tie_embeddings
    return cfg


def lat_model_config_json(vocab_size, hidden_dim, n_layers, n_heads, max_seq_len, latent_dim, rope_dim, nope_dim,
                          v_dim, n_experts, top_k, expert_dim, n_shared, rope_theta=10000.0, norm_eps=1e-5,
                          fine_grained_factor=1, mla_heads=None, tie_embeddings=True, **_formats):
    """ModelConfig of an MLA + MoE decoder (config.rs:732-776 with MoeConfig :99-130,
    HybridAttentionSchedule :626-654 listing every layer in mla_layers, MlaConfig :529-556)
    as serde_json writes it.  n_heads is the transformer's head count and, unless mla_heads
    is given, the MLA head count too; n_experts routed fine experts come from
    n_experts / fine_grained_factor coarse experts of width expert_dim * fine_grained_factor."""
    assert n_experts % fine_grained_factor == 0
    return {
        "vocab_size": vocab_size, "hidden_dim": hidden_dim, "ffn_dim": 4 * hidden_dim, "n_layers": n_layers,
        "n_heads": n_heads, "n_kv_heads": n_heads, "max_seq_len": max_seq_len, "rope_theta": rope_theta,
        "moe": {"num_experts": n_experts // fine_grained_factor, "top_k": top_k,
                "expert_ffn_dim": expert_dim * fine_grained_factor, "aux_loss_weight": 0.01, "every_n_layers": 1,
                "fine_grained_factor": fine_grained_factor, "num_shared_experts": n_shared},
        "attention_schedule": {
            "full_attention_every_n": 4,
            "gated_deltanet": {"n_heads": 0, "key_head_dim": 0, "value_head_dim": 0, "conv_kernel_size": 4,
                               "chunk_size": 64},
            "mla_layers": list(range(n_layers)),
            "mla": {"latent_dim": latent_dim, "nope_head_dim": nope_dim, "rope_head_dim": rope_dim,
                    "n_heads": n_heads if mla_heads is None else mla_heads, "value_head_dim": v_dim}},
        "norm_eps": norm_eps,
        "tie_embeddings": tie_embeddings,
    }


def save_gguf(path, config, fmt, tensors):
    """save_gguf (gguf.rs:47-72): magic, version, JSON metadata, tensors sorted by name,
    each with its shape, encoding byte and payload."""
    meta = json.dumps({"config": config, "format": fmt}, separators=(",", ":")).encode()
    with open(path, "wb") as f:
        f.write(MAGIC)
        f.write(struct.pack("<I", VERSION))
        f.write(struct.pack("<Q", len(meta)))
        f.write(meta)
        f.write(struct.pack("<Q", len(tensors)))
        for name in sorted(tensors):
            arr = np.asarray(tensors[name], np.float32)
            nb = name.encode()
            f.write(struct.pack("<Q", len(nb)))
            f.write(nb)
            f.write(struct.pack("<Q", arr.ndim))
            for d in arr.shape:
                f.write(struct.pack("<Q", d))
            enc = encoding_for(name, arr.shape, fmt)
            payload = encode_tensor(enc, arr)
            f.write(bytes([enc]))
            f.write(struct.pack("<Q", len(payload)))
            f.write(payload)


def load_gguf_tensors(path):
    """load_gguf_tensors (gguf.rs:91-125): (metadata dict, {name: f32 array})."""
    with open(path, "rb") as f:
        data = f.read()
    if data[:4] != MAGIC:
        raise ValueError("not an Aarambh GGUF file")
    (version,) = struct.unpack_from("<I", data, 4)
    if version != VERSION:
        raise ValueError(f"unsupported GGUF version {version}, expected {VERSION}")
    (mlen,) = struct.unpack_from("<Q", data, 8)
    off = 16
    meta = json.loads(data[off:off + mlen].decode())
    off += mlen
    (count,) = struct.unpack_from("<Q", data, off)
    off += 8
    out = {}
    for _ in range(count):
        (nl,) = struct.unpack_from("<Q", data, off)
        off += 8
        name = data[off:off + nl].decode()
        off += nl
        (nd,) = struct.unpack_from("<Q", data, off)
        off += 8
        shape = struct.unpack_from("<" + "Q" * nd, data, off)
        off += 8 * nd
        enc = data[off]
        off += 1
        (pl,) = struct.unpack_from("<Q", data, off)
        off += 8
        out[name] = decode_tensor(enc, shape, data[off:off + pl])
        off += pl
    return meta, out


def save_safetensors(path, tensors, dtype="F32", metadata=None):
    """A safetensors file (candle_core::safetensors::save in save_model, lib.rs:68-71):
    8-byte header length, JSON header {name: {dtype, shape, data_offsets}}, data."""
    header, blobs, off = {}, [], 0
    for name in sorted(tensors):
        arr = np.asarray(tensors[name], np.float32)
        if dtype == "F32":
            raw = arr.astype("<f4").tobytes()
        elif dtype == "F16":
            raw = arr.astype("<f2").tobytes()
        elif dtype == "BF16":
            b = arr.view(np.uint32).astype(np.uint64)
            rne = ((b + 0x7FFF + ((b >> 16) & 1)) >> 16).astype(np.uint16)
            raw = rne.astype("<u2").tobytes()
        else:
            raise ValueError(dtype)
        header[name] = {"dtype": dtype, "shape": list(arr.shape), "data_offsets": [off, off + len(raw)]}
        blobs.append(raw)
        off += len(raw)
    if metadata:
        header["__metadata__"] = metadata
    h = json.dumps(header, separators=(",", ":")).encode()
    h += b" " * ((8 - len(h) % 8) % 8)
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(h)))
        f.write(h)
        for b in blobs:
            f.write(b)


def safetensors_values(tensors, dtype):
    """The f32 values a reader obtains from save_safetensors(tensors, dtype)."""
    out = {}
    for name, arr in tensors.items():
        a = np.asarray(arr, np.float32)
        if dtype == "F16":
            a = a.astype(np.float16).astype(np.float32)
        elif dtype == "BF16":
            b = a.view(np.uint32).astype(np.uint64)
            rne = ((b + 0x7FFF + ((b >> 16) & 1)) >> 16).astype(np.uint32)
            a = (rne << 16).astype(np.uint32).view(np.float32)
        out[name] = a
    return out
