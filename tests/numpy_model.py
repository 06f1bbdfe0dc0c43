"""Float64 numpy statement of the talker / predictor math, vectorised and
written from the reference's definitions (src/talker.rs:263-360,
src/code_predictor.rs:218-273, src/rope.rs:11-93, src/gemv.rs:406-451).

Test infrastructure: an independent second statement used to pin the C
oracle's composite paths (index order, GQA head map, split-half RoPE pairs,
causal masks, residual wiring) on small shapes.  It shares no code with the
oracle: matrices are dequantized once and applied with float64 matmuls.
"""
import numpy as np


def f16(bits):
    return np.asarray(bits, dtype=np.uint16).view(np.float16).astype(np.float64)


def dequant(w):
    """Q4 [k][n] -> float64 matrix ((nib - 8) * scale)."""
    return w.dequantize().astype(np.float64)


def rms_norm(x, gamma_bits, eps=1e-6):
    x = np.asarray(x, dtype=np.float64)
    return x / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + eps) * f16(gamma_bits)


def rope_angles(head_dim, pos, theta):
    i = np.arange(head_dim // 2, dtype=np.float64)
    freq = 1.0 / theta ** (2.0 * i / head_dim)
    ang = np.float64(pos) * freq
    return np.cos(ang), np.sin(ang)


def rope(x, pos, theta):
    """x: [heads, head_dim]; pairs (i, i + head_dim/2)."""
    hd = x.shape[-1]
    c, s = rope_angles(hd, pos, theta)
    x1, x2 = x[..., : hd // 2], x[..., hd // 2:]
    return np.concatenate([x1 * c - x2 * s, x2 * c + x1 * s], axis=-1)


def silu(x):
    return x / (1.0 + np.exp(-x))


def attention(q, k, v):
    """q: [nq, hd]; k, v: [L, nkv, hd] -> [nq, hd] (GQA: head h uses kv h // (nq/nkv))."""
    nq, hd = q.shape
    nkv = k.shape[1]
    g = nq // nkv
    out = np.empty_like(q)
    for h in range(nq):
        kh = h // g
        sc = (k[:, kh, :] @ q[h]) / np.sqrt(hd)
        p = np.exp(sc - sc.max())
        p /= p.sum()
        out[h] = p @ v[:, kh, :]
    return out


class Stack:
    """A layer stack (talker or predictor) with dequantized float64 weights."""

    def __init__(self, layers, cfg):
        self.cfg = cfg
        self.L = []
        for lw in layers:
            self.L.append(dict(q=dequant(lw.q_proj), k=dequant(lw.k_proj), v=dequant(lw.v_proj),
                               o=dequant(lw.o_proj), gate=dequant(lw.gate_proj), up=dequant(lw.up_proj),
                               down=dequant(lw.down_proj), qn=lw.q_norm, kn=lw.k_norm,
                               g_in=lw.input_norm_gamma, g_post=lw.post_attn_norm_gamma))

    def step(self, x, cache, pos):
        """One token through every layer.  cache: list of (K [L,nkv,hd], V)
        per layer, extended in place.  Returns the residual stream."""
        c = self.cfg
        x = np.asarray(x, dtype=np.float64).copy()
        for i, W in enumerate(self.L):
            xn = rms_norm(x, W["g_in"])
            q = (xn @ W["q"]).reshape(c.heads, c.head_dim)
            k = (xn @ W["k"]).reshape(c.kv_heads, c.head_dim)
            v = (xn @ W["v"]).reshape(c.kv_heads, c.head_dim)
            q = rope(rms_norm(q, W["qn"]), pos, c.rope_theta)
            k = rope(rms_norm(k, W["kn"]), pos, c.rope_theta)
            K, V = cache[i]
            K = np.concatenate([K, k[None]], axis=0)
            V = np.concatenate([V, v[None]], axis=0)
            cache[i] = (K, V)
            a = attention(q, K, V).reshape(-1)
            x = x + a @ W["o"]
            xn = rms_norm(x, W["g_post"])
            x = x + (silu(xn @ W["gate"]) * (xn @ W["up"])) @ W["down"]
        return x

    def empty_cache(self):
        c = self.cfg
        z = np.zeros((0, c.kv_heads, c.head_dim))
        return [(z.copy(), z.copy()) for _ in self.L]


class TalkerModel:
    def __init__(self, tw):
        self.cfg = tw.cfg
        self.stack = Stack(tw.layers, tw.cfg)
        self.head = dequant(tw.codec_head)
        self.emb = dequant(tw.codec_embedding)
        self.final = tw.final_norm_gamma

    def forward_with_embedding(self, emb, cache, pos):
        x = self.stack.step(emb, cache, pos)
        h = rms_norm(x, self.final)
        return np.concatenate([h, h @ self.head])

    def prefill(self, X, cache):
        """Causal prefill from position 0 == one step per token."""
        for t in range(X.shape[0]):
            x = self.stack.step(X[t], cache, t)
        return rms_norm(x, self.final)


class PredictorModel:
    def __init__(self, pw):
        self.cfg = pw.cfg
        self.stack = Stack(pw.layers, pw.cfg)
        self.in_proj = dequant(pw.input_proj)
        self.bias = pw.input_proj_bias.astype(np.float64)
        self.embs = [dequant(e) for e in pw.codec_embeddings]
        self.heads = [dequant(h) for h in pw.lm_heads]
        self.final = pw.final_norm_gamma
        self.groups = pw.num_groups

    def project(self, x):
        return np.asarray(x, dtype=np.float64) @ self.in_proj + self.bias

    def generate_acoustic_codes(self, talker_hidden, semantic):
        cache = self.stack.empty_cache()
        self.stack.step(self.project(talker_hidden), cache, 0)
        x = self.stack.step(self.project(semantic), cache, 1)
        logits = [rms_norm(x, self.final) @ self.heads[0]]
        codes = [int(np.argmax(logits[0]))]
        for g in range(1, self.groups):
            x = self.stack.step(self.project(self.embs[g - 1][codes[-1]]), cache, g + 1)
            logits.append(rms_norm(x, self.final) @ self.heads[g])
            codes.append(int(np.argmax(logits[-1])))
        return np.array(codes, dtype=np.uint32), logits
