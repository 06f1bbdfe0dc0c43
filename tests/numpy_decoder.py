"""Float64 statement of the speech decoder's mathematics, vectorised with
numpy and written from the reference's definitions (src/decoder.rs:142-602,
src/conv.rs:151-455): the independent check the oracle's decoder restatement
is pinned against.  Signals are channel-first [C][L]; transformer rows are
token-major [T][D]; projection weights are [in][out] (y = x @ W)."""
import numpy as np


def f64(a):
    return np.asarray(a, dtype=np.float64)


def causal_conv(x, w, b, dilation=1):
    """CausalConv1d (src/conv.rs:151-184): x [Cin][L], w [Cout][Cin][K]; left
    padding (K-1)*dilation, output length L."""
    x, w, b = f64(x), f64(w), f64(b)
    cout, cin, k = w.shape
    L = x.shape[1]
    pad = (k - 1) * dilation
    xp = np.concatenate([np.zeros((cin, pad)), x], axis=1)
    out = np.repeat(b[:, None], L, axis=1)
    for t in range(k):
        out = out + w[:, :, t] @ xp[:, t * dilation: t * dilation + L]
    return out


def transposed_conv(x, w, b, stride, padding=0, crop=True):
    """ConvTranspose1d (src/conv.rs:197-268): x [Cin][L], w [Cin][Cout][K];
    out[(i*stride + k - padding)] += x[i] * w[k]; then the decoder's causal
    right crop of K - stride samples (src/decoder.rs:430-444)."""
    x, w, b = f64(x), f64(w), f64(b)
    cin, cout, k = w.shape
    L = x.shape[1]
    full = (L - 1) * stride - 2 * padding + k
    out = np.repeat(b[:, None], full, axis=1)
    for t in range(k):
        pos = np.arange(L) * stride + t - padding
        ok = (pos >= 0) & (pos < full)
        contrib = w[:, :, t].T @ x  # [Cout][L]
        np.add.at(out, (slice(None), pos[ok]), contrib[:, ok])
    if crop and k - stride > 0:
        out = out[:, : full - (k - stride)]
    return out


def depthwise_conv(x, w, b):
    """DepthwiseConv1d (src/conv.rs:297-345): causal, left padding K-1 whatever
    the weight's padding field; x [C][L], w [C][K]."""
    x, w, b = f64(x), f64(w), f64(b)
    c, k = w.shape
    L = x.shape[1]
    xp = np.concatenate([np.zeros((c, k - 1)), x], axis=1)
    out = np.repeat(b[:, None], L, axis=1)
    for t in range(k):
        out = out + w[:, t: t + 1] * xp[:, t: t + L]
    return out


def snake(x, alpha, beta):
    """SnakeBeta (src/conv.rs:346-400): x + exp(-beta) * sin(exp(alpha) * x)^2."""
    x = f64(x)
    a = np.exp(f64(alpha))[:, None]
    return x + np.exp(-f64(beta))[:, None] * np.sin(a * x) ** 2


def gelu(x):
    """The decoder's GELU (src/conv.rs:452-455): x * 0.5 * (1 + tanh(x / sqrt 2))."""
    x = f64(x)
    return x * 0.5 * (1.0 + np.tanh(x / np.sqrt(2.0)))


def layer_norm_cf(x, g, b, eps=1e-5):
    """LayerNorm over channels at each time step (src/decoder.rs:580-602)."""
    x = f64(x)
    mean = x.mean(axis=0, keepdims=True)
    var = ((x - mean) ** 2).mean(axis=0, keepdims=True)
    return (x - mean) / np.sqrt(var + eps) * f64(g)[:, None] + f64(b)[:, None]


def rms_norm(x, g, eps=1e-5):
    """rms_norm_f32 (src/decoder.rs:515-525) over the last axis."""
    x = f64(x)
    return x / np.sqrt((x * x).mean(axis=-1, keepdims=True) + eps) * f64(g)


def rope_split_half(x, heads, hd, pos, cos_t, sin_t):
    """apply_rope_split_half (src/decoder.rs:556-578): pairs (i, i + hd/2);
    no rotation at positions past the table."""
    x = f64(x).reshape(heads, hd).copy()
    half = hd // 2
    cos_t, sin_t = f64(cos_t).reshape(-1, half), f64(sin_t).reshape(-1, half)
    if pos >= cos_t.shape[0]:
        return x.reshape(-1)
    c, s = cos_t[pos], sin_t[pos]
    x0, x1 = x[:, :half].copy(), x[:, half:].copy()
    x[:, :half] = x0 * c - x1 * s
    x[:, half:] = x1 * c + x0 * s
    return x.reshape(-1)


def window_attention(q, k, v, heads, hd, window):
    """Causal sliding-window attention (src/decoder.rs:262-300): q, k, v
    [T][heads*hd]; row t attends to max(0, t+1-window) .. t."""
    q, k, v = f64(q), f64(k), f64(v)
    T = q.shape[0]
    out = np.zeros_like(q)
    for t in range(T):
        s0 = max(0, t + 1 - window)
        for h in range(heads):
            sl = slice(h * hd, (h + 1) * hd)
            sc = k[s0: t + 1, sl] @ q[t, sl] / np.sqrt(hd)
            p = np.exp(sc - sc.max())
            p /= p.sum()
            out[t, sl] = p @ v[s0: t + 1, sl]
    return out


def codebook_lookup(w, codes):
    """codebook_lookup (src/decoder.rs:142-189): [vq_dim][T]."""
    c = w.cfg
    cd, vq = c.codebook_dim, c.vq_dim
    cb0 = f64(w.first_codebook).reshape(c.codebook_size, cd)
    p0 = f64(w.first_output_proj).reshape(cd, vq)
    pr = f64(w.rest_output_proj).reshape(cd, vq)
    first = cb0[codes[0]] @ p0
    rest = sum(f64(w.rest_codebooks[g]).reshape(c.codebook_size, cd)[codes[g + 1]] for g in range(c.num_rest))
    return (first + rest @ pr).T


def _conv(d):
    k = d["kernel_size"]
    return f64(d["weight"]).reshape(d["out_channels"], d["in_channels"], k), d["bias"], d["dilation"]


def _tconv(d):
    return (f64(d["weight"]).reshape(d["in_channels"], d["out_channels"], d["kernel_size"]), d["bias"],
            d["stride"], d["padding"])


def transformer(w, x_ch):
    """decoder_transformer (src/decoder.rs:195-330): [latent][T] -> [latent][T]."""
    c = w.cfg
    hid, ad, lat = c.hidden, c.heads * c.head_dim, c.latent
    T = x_ch.shape[1]
    x = f64(x_ch).T @ f64(w.tf_input_w).reshape(lat, hid) + f64(w.tf_input_b)
    for L in w.layers:
        xn = rms_norm(x, L["input_norm"])
        q = xn @ f64(L["q_proj"]).reshape(hid, ad)
        k = xn @ f64(L["k_proj"]).reshape(hid, ad)
        v = xn @ f64(L["v_proj"]).reshape(hid, ad)
        q = np.stack([rope_split_half(q[t], c.heads, c.head_dim, t, w.rope_cos, w.rope_sin) for t in range(T)])
        k = np.stack([rope_split_half(k[t], c.heads, c.head_dim, t, w.rope_cos, w.rope_sin) for t in range(T)])
        a = window_attention(q, k, v, c.heads, c.head_dim, c.window)
        x = x + (a @ f64(L["o_proj"]).reshape(ad, hid)) * f64(L["attn_scale"])
        xn = rms_norm(x, L["post_attn_norm"])
        g = xn @ f64(L["gate_proj"]).reshape(hid, c.inter)
        u = xn @ f64(L["up_proj"]).reshape(hid, c.inter)
        h = g / (1.0 + np.exp(-g)) * u
        x = x + (h @ f64(L["down_proj"]).reshape(c.inter, hid)) * f64(L["mlp_scale"])
    x = rms_norm(x, w.tf_norm)
    return (x @ f64(w.tf_output_w).reshape(hid, lat) + f64(w.tf_output_b)).T


def convnext(x, st):
    """convnext_forward (src/decoder.rs:336-388)."""
    ch = x.shape[0]
    dw = st["dw_conv"]
    y = depthwise_conv(x, f64(dw["weight"]).reshape(ch, dw["kernel_size"]), dw["bias"])
    y = layer_norm_cf(y, st["norm_w"], st["norm_b"])
    inner = st["inner"]
    h = gelu(y.T @ f64(st["pw1_w"]).reshape(ch, inner) + f64(st["pw1_b"]))
    z = h @ f64(st["pw2_w"]).reshape(inner, ch) + f64(st["pw2_b"])
    return f64(x) + f64(st["gamma"])[:, None] * z.T


def decode_to_audio(w, codes):
    """decode_to_audio (src/decoder.rs:394-509), float64; the final clamp to
    [-1, 1] included."""
    x = codebook_lookup(w, codes)
    x = causal_conv(x, *_conv(w.pre_conv))
    x = transformer(w, x)
    for st in w.upsample:
        wt, b, s, p = _tconv(st["conv_t"])
        x = transposed_conv(x, wt, b, s, p)
        x = convnext(x, st)
    x = causal_conv(x, *_conv(w.vocos_init))
    for blk in w.blocks:
        x = snake(x, blk["pre_snake_alpha"], blk["pre_snake_beta"])
        wt, b, s, p = _tconv(blk["upsample"])
        x = transposed_conv(x, wt, b, s, p)
        for r in blk["residuals"]:
            y = snake(x, r["act1_alpha"], r["act1_beta"])
            y = causal_conv(y, *_conv(r["conv1"]))
            y = snake(y, r["act2_alpha"], r["act2_beta"])
            y = causal_conv(y, *_conv(r["conv2"]))
            x = x + y
    x = snake(x, w.final_snake_alpha, w.final_snake_beta)
    x = causal_conv(x, *_conv(w.output_conv))
    return np.clip(x.reshape(-1), -1.0, 1.0)
