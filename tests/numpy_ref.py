"""Independent float64 numpy forward of the Llama-2 / Stories model (test helper).

Vectorised, written from the model definition rather than from the oracle's
loops: RMSNorm with eps inside the root, interleaved-pair RoPE with
theta_i = pos * 10000^(-2i/hd), causal softmax attention scaled by 1/sqrt(hd),
SwiGLU FFN, pre-norm residuals, final norm and classifier
(training/forward.h:104-170).  Used to cross-check the oracle's composition.
"""
import numpy as np


def split_weights(cfg7, w, untied):
    D, F, L, H, Hkv, V = cfg7[0], cfg7[1], cfg7[2], cfg7[3], cfg7[4], abs(cfg7[5])
    hd = D // H
    NQ, NKV = H * hd, Hkv * hd
    w = np.asarray(w, dtype=np.float64)
    sizes = [("embed", (V, D)), ("rms_att", (L, D)), ("wq", (L, NQ, D)), ("wk", (L, NKV, D)),
             ("wv", (L, NKV, D)), ("wo", (L, D, NQ)), ("rms_ffn", (L, D)), ("w1", (L, F, D)),
             ("w2", (L, D, F)), ("w3", (L, F, D)), ("rms_final", (D,))]
    if untied:
        sizes.append(("wcls", (V, D)))
    out, off = {}, 0
    for name, shp in sizes:
        n = int(np.prod(shp))
        out[name] = w[off:off + n].reshape(shp)
        off += n
    assert off == w.size
    if not untied:
        out["wcls"] = out["embed"]
    return out


def forward(cfg7, w, untied, tokens):
    D, L, H, Hkv = cfg7[0], cfg7[2], cfg7[3], cfg7[4]
    hd = D // H
    P = split_weights(cfg7, w, untied)
    S = len(tokens)
    x = P["embed"][np.asarray(tokens)]
    pos = np.arange(S)[:, None]
    theta = pos * 10000.0 ** (-np.arange(0, hd, 2) / hd)[None]
    c, s = np.cos(theta), np.sin(theta)

    def rms(v, g):
        return v / np.sqrt((v * v).mean(-1, keepdims=True) + 1e-5) * g

    def rope(a, nh):
        a = a.reshape(S, nh, hd // 2, 2)
        e, o = a[..., 0], a[..., 1]
        return np.stack([e * c[:, None] - o * s[:, None], e * s[:, None] + o * c[:, None]], -1).reshape(S, nh * hd)

    mask = np.triu(np.full((S, S), -np.inf), 1)
    for l in range(L):
        xn = rms(x, P["rms_att"][l])
        q = rope(xn @ P["wq"][l].T, H).reshape(S, H, hd)
        k = rope(xn @ P["wk"][l].T, Hkv).reshape(S, Hkv, hd)
        v = (xn @ P["wv"][l].T).reshape(S, Hkv, hd)
        rep = H // Hkv
        k = np.repeat(k, rep, axis=1)
        v = np.repeat(v, rep, axis=1)
        sc = np.einsum("thd,shd->hts", q, k) / np.sqrt(hd) + mask
        p = np.exp(sc - sc.max(-1, keepdims=True))
        p /= p.sum(-1, keepdims=True)
        att = np.einsum("hts,shd->thd", p, v).reshape(S, H * hd)
        x = x + att @ P["wo"][l].T
        xn = rms(x, P["rms_ffn"][l])
        h1, h3 = xn @ P["w1"][l].T, xn @ P["w3"][l].T
        x = x + (h1 / (1 + np.exp(-h1)) * h3) @ P["w2"][l].T
    return rms(x, P["rms_final"]) @ P["wcls"].T
