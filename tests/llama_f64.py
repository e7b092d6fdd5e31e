"""A float64 restatement of one Llama-3 decode step, written from the model's
equations, independent of the C oracle (oracle/qorus_oracle.c).

It pins or_decode_step's composition: which norm feeds which projection, the
residual order, the RoPE pairing and position, the GQA head mapping and the
cache rows attended.  The numerics follow the reference's own definitions
where they differ from textbook ones -- the clamped degree-5 polynomial exp
(reference src/ops/avx2/avx_math.h:10-61) on the first len&~7 elements of
softmax and SiLU and libm exp on the rest (softmax.c:182-196,
silu.c:44-51) -- but every value is carried in float64:

    x = E[token]
    per layer l:
        h  = x / sqrt(mean(x^2) + eps) * w_attn[l]          (rmsnorm.c:15-92)
        q, k, v = Wq h, Wk h, Wv h                          (model.c:1110-1165)
        RoPE on each head, GPT-J pairs (2i, 2i+1),
            theta_i = pos * base^(-2i/head_dim)             (rope.c:23-110, model.c:633-659)
        cache[l][kv_head][pos] = (k_rot, v)                 (model.c:700-740)
        head h attends kv head h // (n_heads / n_kv) over positions 0..pos:
            p = softmax(q_h . k_j / sqrt(head_dim)),  o_h = sum_j p_j v_j
        x1 = x + Wo o                                        (model.c:1450, 1620)
        h2 = x1 / sqrt(mean(x1^2) + eps) * w_ffn[l]          (model.c:1624)
        x  = x1 + Wd (silu(Wg h2) * (Wu h2))                 (model.c:1465-1564, 1647)
    logits = W_lm (x / sqrt(mean(x^2) + eps) * w_out)        (model.c:1799-1844)
    token  = first index of the largest logit                (main.c:870-881)

with [out, in] matrices and a Q4_0 LM head (the build's corrected shapes).
`mistake` plants one wrong composition step, so a test can show that the
comparison catches it.
"""
from __future__ import annotations

import math

import numpy as np

from oracle import oracle as orc

# Reference polynomial coefficients (float32 literals of avx_math.h).
_C = [1.0, 1.0, 0.5] + [float(np.float32(v)) for v in (0.16666667, 0.04166667, 0.00833333)]


def exp_poly(x: float) -> float:
    if x < -10.0:
        return 0.0
    if x > 10.0:
        return 22026.0
    t = min(max(x, -5.0), 5.0)
    return max(sum(c * t ** i for i, c in enumerate(_C)), 0.0)


def ref_exp_row(d: np.ndarray) -> np.ndarray:
    """The reference's exp over a vector: the polynomial on the first
    len&~7 entries, libm exp on the rest (all libm when len < 8)."""
    n = len(d)
    nv = n & ~7 if n >= 8 else 0
    return np.array([exp_poly(float(v)) if i < nv else math.exp(float(v)) for i, v in enumerate(d)])


def rms(x, w, eps):
    return x / math.sqrt(float(np.mean(x * x)) + eps) * w


def silu(g):
    return g / (1.0 + ref_exp_row(-g))


def rope(v, pos, base, hd, n_heads, rotate_half=False):
    out = np.empty_like(v)
    i = np.arange(hd // 2)
    th = pos * np.power(float(base), -2.0 * i / hd)
    c, s = np.cos(th), np.sin(th)
    for h in range(n_heads):
        u = v[h * hd:(h + 1) * hd]
        if rotate_half:  # the other common pairing (i, i + hd/2): a planted mistake
            a, b = u[:hd // 2], u[hd // 2:]
            out[h * hd:h * hd + hd // 2] = a * c - b * s
            out[h * hd + hd // 2:(h + 1) * hd] = b * c + a * s
        else:
            a, b = u[0::2], u[1::2]
            out[h * hd:(h + 1) * hd:2] = a * c - b * s
            out[h * hd + 1:(h + 1) * hd:2] = b * c + a * s
    return out


class Llama64:
    """The model of a .qorus v3 blob in float64 (weights dequantized as
    (q - 8) * s exactly), with its own float64 KV cache."""

    def __init__(self, blob: np.ndarray, kv32: np.ndarray):
        h = orc.parse_header(blob)
        self.h = h
        lay = orc.model_layout(h)
        D, H, V, L = h["dim"], h["hidden"], h["vocab"], h["n_layers"]
        self.hd = D // h["n_heads"]
        kvd = h["n_kv"] * self.hd

        def f32(name, n):
            o = lay[name]
            return blob[o:o + 4 * n].view(np.float32).astype(np.float64)

        def q4(name, rows, cols):
            o = lay[name]
            return orc.dequant_np(blob[o:o + rows * (cols // 32) * 20].reshape(rows, -1))

        self.embd = f32("token_embd", V * D).reshape(V, D)
        self.w_out = f32("output_norm", D)
        self.lm = q4("output", V, D)
        self.layers = []
        for l in range(L):
            self.layers.append(dict(
                attn_norm=f32(f"{l}.attn_norm", D), ffn_norm=f32(f"{l}.ffn_norm", D),
                wq=q4(f"{l}.wq", D, D), wk=q4(f"{l}.wk", kvd, D), wv=q4(f"{l}.wv", kvd, D),
                wo=q4(f"{l}.wo", D, D), wg=q4(f"{l}.w_gate", H, D), wu=q4(f"{l}.w_up", H, D),
                wd=q4(f"{l}.w_down", D, H)))
        self.kv = kv32.astype(np.float64)  # [L][n_kv][max_seq][2][hd]

    def step(self, token: int, pos: int, mistake: str = ""):
        h = self.h
        D, nh, nkv, hd, eps = h["dim"], h["n_heads"], h["n_kv"], self.hd, h["eps"]
        base = h["rope_base"]
        group = nh // nkv
        x = self.embd[token].copy()
        for l, w in enumerate(self.layers):
            hn = rms(x, w["ffn_norm"] if mistake == "norm_weight" else w["attn_norm"], eps)
            q, k, v = w["wq"] @ hn, w["wk"] @ hn, w["wv"] @ hn
            rp = pos + 1 if mistake == "rope_pos" else pos
            half = mistake == "rope_pairs"
            q, k = rope(q, rp, base, hd, nh, half), rope(k, rp, base, hd, nkv, half)
            for kh in range(nkv):
                self.kv[l, kh, pos, 0] = k[kh * hd:(kh + 1) * hd]
                self.kv[l, kh, pos, 1] = v[kh * hd:(kh + 1) * hd]
            o = np.empty(D)
            for hh in range(nh):
                kvh = hh % nkv if mistake == "gqa" else hh // group
                K = self.kv[l, kvh, :pos + 1, 0]
                Vv = self.kv[l, kvh, :pos + 1, 1]
                s = K @ q[hh * hd:(hh + 1) * hd] / math.sqrt(hd)
                e = ref_exp_row(s - s.max())
                o[hh * hd:(hh + 1) * hd] = (e / e.sum()) @ Vv
            x1 = x + w["wo"] @ o
            h2 = rms(x1, w["ffn_norm"], eps)
            m = silu(w["wg"] @ h2) * (w["wu"] @ h2)
            x = (x if mistake == "residual" else x1) + w["wd"] @ m
        logits = self.lm @ rms(x, self.w_out, eps)
        return int(np.argmax(logits)), logits
