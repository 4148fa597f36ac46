"""Float64 textbook formulation of the Qwen3.5/3.6 hybrid decode step, used to
pin the CPU restatement's semantics (not its rounding): gated delta rule with
the GGUF key-head mapping (value head h reads key head h % KH,
cached_delta.hex:77-79), 4-tap causal conv with SiLU, per-head L2 norms,
gated RMSNorm, partial neox RoPE, gated GQA attention with a sigmoid output
gate, SwiGLU or a top-k softmax-renormalised MoE with a sigmoid-gated shared
expert. Weights are the same BF16/F32 tensors; activations stay in float64."""
from __future__ import annotations

import numpy as np


def bf(a):
    a = np.asarray(a)
    if a.dtype == np.uint16:
        return (a.astype(np.uint32) << 16).view(np.float32).astype(np.float64)
    return a.astype(np.float64)


def silu(x):
    return x / (1.0 + np.exp(-x))


def sigmoid(x):
    return 1.0 / (1.0 + np.exp(-x))


def softplus(x):
    return np.maximum(x, 0) + np.log1p(np.exp(-np.abs(x)))


def rms(x, w, eps):
    return x / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + eps) * w


class Textbook:
    def __init__(self, cfg, weights, key_head=lambda h, KH, VH: h % KH):
        self.c = cfg
        self.w = weights
        self.key_head = key_head
        c = cfg
        self.full = [(l + 1) % c["full_interval"] == 0 for l in range(c["layers"])]
        self.base = []
        b = 1
        for l in range(c["layers"]):
            self.base.append(b)
            b += (16 if c["moe"] else 11) if self.full[l] else (19 if c["moe"] else 14)
        self.KS = c["key_heads"] * c["key_dim"]
        self.VS = c["value_heads"] * c["value_dim"]
        self.QKV = 2 * self.KS + self.VS
        self.reset()

    def reset(self):
        c = self.c
        self.hist = [np.zeros((0, self.QKV)) for _ in range(c["layers"])]
        self.S = [np.zeros((c["value_heads"], c["value_dim"], c["key_dim"])) for _ in range(c["layers"])]
        self.K = [[] for _ in range(c["layers"])]
        self.V = [[] for _ in range(c["layers"])]

    def import_cache(self, cache, capacity, position):
        """Take over a BF16 session state in the reference layout
        (src/spec.rs:321-362): K/V rows of positions < position, the conv
        history of positions position-3 .. position-1 (slot p mod 3) and the
        DeltaNet state."""
        c = self.c
        KVS = c["kv_heads"] * c["head_dim"]
        kv = bf(cache[:c["layers"] * 2 * capacity * KVS]).reshape(c["layers"], 2, capacity,
                                                                    c["kv_heads"], c["head_dim"])
        tail = bf(cache[c["layers"] * 2 * capacity * KVS:]).reshape(c["layers"], -1)
        conv = 3 * self.QKV
        for l in range(c["layers"]):
            self.K[l] = [kv[l, 0, p] for p in range(position)]
            self.V[l] = [kv[l, 1, p] for p in range(position)]
            slots = tail[l, :conv].reshape(3, self.QKV)
            rows = [slots[(position + t) % 3] for t in range(3) if position - 3 + t >= 0]
            self.hist[l] = np.array(rows).reshape(-1, self.QKV)
            self.S[l] = tail[l, conv:].reshape(c["value_heads"], c["value_dim"], c["key_dim"]).copy()

    def W(self, l, s, rows=None, cols=None):
        a = bf(self.w[self.base[l] + s])
        if rows is not None:
            a = a.reshape(rows, cols)
        return a

    def step(self, token, pos):
        c = self.c
        H, HD, R = c["hidden"], c["head_dim"], c["rope_dim"]
        h = bf(self.w[0]).reshape(c["vocab"], H)[token].copy()
        for l in range(c["layers"]):
            x = rms(h, self.W(l, 0), c["eps"])
            if self.full[l]:
                Q, KVH = c["q_heads"], c["kv_heads"]
                qg = (self.W(l, 1, 2 * Q * HD, H) @ x).reshape(Q, 2, HD)
                q, gate = qg[:, 0], qg[:, 1]
                k = (self.W(l, 2, KVH * HD, H) @ x).reshape(KVH, HD)
                v = (self.W(l, 3, KVH * HD, H) @ x).reshape(KVH, HD)
                q = rms(q, self.W(l, 5), c["eps"])
                k = rms(k, self.W(l, 6), c["eps"])
                half = R // 2
                freq = np.float64(c["theta"]) ** (-(2.0 * np.arange(half)) / R)
                ang = pos * freq
                cos, sin = np.cos(ang), np.sin(ang)

                def rope(t):
                    t = t.copy()
                    a, b = t[..., :half].copy(), t[..., half:R].copy()
                    t[..., :half] = a * cos - b * sin
                    t[..., half:R] = b * cos + a * sin
                    return t

                q, k = rope(q), rope(k)
                self.K[l].append(k)
                self.V[l].append(v)
                Ks, Vs = np.stack(self.K[l]), np.stack(self.V[l])
                out = np.zeros((Q, HD))
                for hh in range(Q):
                    kv = hh // (Q // KVH)
                    s = Ks[:, kv] @ q[hh] / np.sqrt(HD)
                    p = np.exp(s - s.max())
                    p /= p.sum()
                    out[hh] = (p @ Vs[:, kv]) * sigmoid(gate[hh])
                attn = h + self.W(l, 4, H, Q * HD) @ out.reshape(-1)
                post, ffn = self.W(l, 7), 8
            else:
                KH, KD, VH, VD = c["key_heads"], c["key_dim"], c["value_heads"], c["value_dim"]
                qkv = self.W(l, 1, self.QKV, H) @ x
                z = self.W(l, 2, self.VS, H) @ x
                a = self.W(l, 3, VH, H) @ x
                b = self.W(l, 4, VH, H) @ x
                conv_w = self.W(l, 9, self.QKV, 4)
                hist = np.vstack([self.hist[l], qkv[None]])
                window = np.zeros((4, self.QKV))
                take = hist[-4:]
                window[4 - len(take):] = take
                conv = silu(np.sum(window.T * conv_w, axis=1))
                self.hist[l] = hist[-3:]
                qh = conv[:self.KS].reshape(KH, KD)
                kh = conv[self.KS:2 * self.KS].reshape(KH, KD)
                vh = conv[2 * self.KS:].reshape(VH, VD)
                qh = qh / np.sqrt(np.sum(qh * qh, axis=1, keepdims=True) + 1e-6)
                kh = kh / np.sqrt(np.sum(kh * kh, axis=1, keepdims=True) + 1e-6)
                dt, A = self.W(l, 5), self.W(l, 6)
                o = np.zeros((VH, VD))
                for hh in range(VH):
                    j = self.key_head(hh, KH, VH)
                    g = np.exp(softplus(a[hh] + dt[hh]) * A[hh])
                    beta = sigmoid(b[hh])
                    S = self.S[l][hh]
                    delta = (vh[hh] - g * (S @ kh[j])) * beta
                    S = g * S + np.outer(delta, kh[j])
                    self.S[l][hh] = S
                    o[hh] = S @ qh[j] / np.sqrt(KD)
                y = rms(o, self.W(l, 7), c["eps"]) * silu(z.reshape(VH, VD))
                attn = h + self.W(l, 8, H, self.VS) @ y.reshape(-1)
                post, ffn = self.W(l, 10), 11
            x = rms(attn, post, c["eps"])
            if c["moe"]:
                E, K, I, SI = c["experts"], c["top_k"], c["intermediate"], c["shared_intermediate"]
                logits = self.W(l, ffn, E, H) @ x
                shared_logit = self.W(l, ffn + 4, 1, H)[0] @ x
                ids = np.argsort(-logits, kind="stable")[:K]
                p = np.exp(logits[ids] - logits[ids[0]])
                p /= p.sum()
                gate = self.W(l, ffn + 1, E * I, H).reshape(E, I, H)
                up = self.W(l, ffn + 2, E * I, H).reshape(E, I, H)
                down = self.W(l, ffn + 3, E * H, I).reshape(E, H, I)
                y = np.zeros(H)
                for j, e in enumerate(ids):
                    y += p[j] * (down[e] @ (silu(gate[e] @ x) * (up[e] @ x)))
                sg, su = self.W(l, ffn + 5, SI, H), self.W(l, ffn + 6, SI, H)
                sd = self.W(l, ffn + 7, H, SI)
                y += sigmoid(shared_logit) * (sd @ (silu(sg @ x) * (su @ x)))
                h = attn + y
            else:
                I = c["intermediate"]
                g = self.W(l, ffn, I, H) @ x
                u = self.W(l, ffn + 1, I, H) @ x
                h = attn + self.W(l, ffn + 2, H, I) @ (silu(g) * u)
        x = rms(h, bf(self.w[-2]), c["eps"])
        return bf(self.w[-1]).reshape(c["vocab"], H) @ x
