"""Float64 numpy forward of the decoder, written from the textbook definitions
(RMSNorm, NeoX half-split RoPE, softmax attention with the interleaved GQA head
map of attention.rs:415-428, SwiGLU).  Used by tests to pin the C oracle; it
shares no code with it (matrix softmax instead of the oracle's online softmax)."""
import numpy as np


def weights(model):
    names = {t[0]: i for i, t in enumerate(model.tensors())}
    return {n: model.get(i).astype(np.float64) for n, i in names.items()}


def rms(x, w, eps):
    return x / np.sqrt((x * x).mean(-1, keepdims=True) + eps) * w.reshape(-1)


def rope(x, pos, theta, rs=None):
    # x [S, H, hd]; rs = (inverse frequencies, cos / sin factor) of a scaled RoPE
    hd = x.shape[-1]
    half = hd // 2
    inv = 1.0 / theta ** (2.0 * np.arange(half) / hd) if rs is None else np.asarray(rs[0], np.float64)
    a = 1.0 if rs is None else float(rs[1])
    ang = pos[:, None] * inv[None, :]
    c, s = a * np.cos(ang)[:, None, :], a * np.sin(ang)[:, None, :]
    x1, x2 = x[..., :half], x[..., half:]
    return np.concatenate([x1 * c - x2 * s, x1 * s + x2 * c], -1)


def block(W, pre, x, cfg, pos, rs=None):
    H, nh, nkv = cfg.hidden_dim, cfg.n_heads, cfg.n_kv_heads
    hd = H // nh
    S = x.shape[0]
    xn = rms(x, W[pre + "norm1.weight"], cfg.norm_eps)
    q = (xn @ W[pre + "attn.wq.weight"].T).reshape(S, nh, hd)
    k = (xn @ W[pre + "attn.wk.weight"].T).reshape(S, nkv, hd)
    v = (xn @ W[pre + "attn.wv.weight"].T).reshape(S, nkv, hd)
    q, k = rope(q, pos, cfg.rope_theta, rs), rope(k, pos, cfg.rope_theta, rs)
    out = np.zeros((S, nh, hd))
    mask = np.tril(np.ones((S, S), bool))
    for h in range(nh):
        kh = h % nkv
        sc = q[:, h] @ k[:, kh].T / np.sqrt(hd)
        sc = np.where(mask, sc, -np.inf)
        p = np.exp(sc - sc.max(-1, keepdims=True))
        p /= p.sum(-1, keepdims=True)
        out[:, h] = p @ v[:, kh]
    x = x + out.reshape(S, nh * hd) @ W[pre + "attn.wo.weight"].T
    xn = rms(x, W[pre + "norm2.weight"], cfg.norm_eps)
    g = xn @ W[pre + "ffn.w_gate.weight"].T
    u = xn @ W[pre + "ffn.w_up.weight"].T
    return x + (g / (1 + np.exp(-g)) * u) @ W[pre + "ffn.w_down.weight"].T


def forward(W, cfg, ids, rs=None):
    """Full (uncached) forward over ids; returns logits [S, V] and normed hidden [S, H].
    rs: (inverse frequencies, cos / sin factor) of a scaled RoPE, None for the base one."""
    E = W["embedding.weight"]
    x = E[np.asarray(ids, np.int64)]
    pos = np.arange(len(ids), dtype=np.float64)
    for l in range(cfg.n_layers):
        x = block(W, f"blocks.{l}.", x, cfg, pos, rs)
    hn = rms(x, W["final_norm.weight"], cfg.norm_eps)
    return hn @ E.T, hn


def mtp_head(W, cfg, head, anchor, ids):
    E = W["embedding.weight"]
    pre = f"mtp.heads.{head}."
    loc = [rms(np.asarray(anchor, np.float64), W[pre + "trunk_norm.weight"], cfg.norm_eps)]
    for t in ids:
        loc.append(rms(E[int(t)], W[pre + "token_norm.weight"], cfg.norm_eps))
    x = np.stack(loc)
    x = block(W, pre + "refine.", x, cfg, np.arange(len(loc), dtype=np.float64))
    return rms(x[-1], W[pre + "output_norm.weight"], cfg.norm_eps) @ E.T


def lat_block(W, pre, x, cfg, pos, absorbed=False):
    """MLA (mla.rs:402-489) + MoE (moe.rs:212-406) block in float64.  The MoE runs
    every expert densely and weights it by the dispatch weight (0 when not
    selected), as the reference does; absorbed=True evaluates attention in the
    latent space (q . up_k c = (up_k^T q) . c, o = up_v (P c)) instead of
    reconstructing K and V."""
    S, H = x.shape
    nh, nope, rd, lat, vd = cfg.n_heads, cfg.nope_dim, cfg.rope_dim, cfg.latent_dim, cfg.v_dim
    xn = rms(x, W[pre + "norm1.weight"], cfg.norm_eps)
    q = (xn @ W[pre + "mla.q_proj.weight"].T).reshape(S, nh, nope + rd)
    qn, qr = q[..., :nope], rope(q[..., nope:], pos, cfg.rope_theta)
    c = rms(xn @ W[pre + "mla.kv_a_proj.weight"].T, W[pre + "mla.kv_a_norm.weight"], cfg.norm_eps)
    kr = rope((xn @ W[pre + "mla.k_rope_proj.weight"].T)[:, None, :], pos, cfg.rope_theta)[:, 0]
    upk = W[pre + "mla.up_k.weight"].reshape(nh, nope, lat)
    upv = W[pre + "mla.up_v.weight"].reshape(nh, vd, lat)
    mask = np.tril(np.ones((S, S), bool))
    out = np.zeros((S, nh, vd))
    for h in range(nh):
        if absorbed:
            ql = qn[:, h] @ upk[h]                      # [S, lat]
            sc = (ql @ c.T + qr[:, h] @ kr.T) / np.sqrt(nope + rd)
        else:
            kn = c @ upk[h].T                            # [T, nope]
            sc = (qn[:, h] @ kn.T + qr[:, h] @ kr.T) / np.sqrt(nope + rd)
        sc = np.where(mask, sc, -np.inf)
        p = np.exp(sc - sc.max(-1, keepdims=True))
        p /= p.sum(-1, keepdims=True)
        out[:, h] = (p @ c) @ upv[h].T if absorbed else p @ (c @ upv[h].T)
    x = x + out.reshape(S, nh * vd) @ W[pre + "mla.o_proj.weight"].T
    xn = rms(x, W[pre + "norm2.weight"], cfg.norm_eps)
    logits = xn @ W[pre + "ffn.router.weight"].T
    E, K = cfg.n_experts, cfg.top_k
    disp = np.zeros((S, E))
    for s in range(S):
        order = sorted(range(E), key=lambda e: (-logits[s, e], e))[:K]
        sel = logits[s, order]
        w = np.exp(sel - sel.max())
        disp[s, order] = w / w.sum()

    def expert(name):
        g = xn @ W[name + "w_gate.weight"].T
        u = xn @ W[name + "w_up.weight"].T
        return (g / (1 + np.exp(-g)) * u) @ W[name + "w_down.weight"].T

    y = sum(expert(pre + f"ffn.experts.{e}.") * disp[:, e:e + 1] for e in range(E))
    for e in range(cfg.n_shared):
        y = y + expert(pre + f"ffn.shared_experts.{e}.")
    return x + y


def lat_forward(W, cfg, ids, absorbed=False):
    E = W["embedding.weight"]
    x = E[np.asarray(ids, np.int64)]
    pos = np.arange(len(ids), dtype=np.float64)
    for l in range(cfg.n_layers):
        x = lat_block(W, f"blocks.{l}.", x, cfg, pos, absorbed)
    hn = rms(x, W["final_norm.weight"], cfg.norm_eps)
    return hn @ E.T, hn
