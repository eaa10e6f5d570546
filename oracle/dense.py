"""Float64 restatement of one dense (Qwen3-style) decode step, the checker for
tbq_dense_decode.

TEST INFRASTRUCTURE ONLY: imported by tests/ (and nothing in the product).

The layer is the model's forward, not the reference's: the reference's
tb_layer_forward (layer4/tb_infer.c:553-883) takes head_dim = hidden /
n_heads when the file gives none, applies RoPE with interleaved pairs
(tb_rope_apply, :142-153) to each K head n_heads / n_kv_heads times, and
applies QK-norm after RoPE.  Here QK-norm comes first, RoPE rotates the
pairs (i, i + D/2) once per head, and head_dim is the model's.  The pieces
that agree with the reference are its rmsnorm (layer1/tb_tensor.c:194-199:
x * (1 / sqrt(mean(x^2) + eps)) * w), its online-softmax GQA attention
(layer1/tb_tensor.c:300-405: kv head = h / (n_heads / n_kv_heads), scale
1/sqrt(D)), SwiGLU (layer4/tb_infer.c:130-135) and the dequantised matvecs
(pinned bit-exact elsewhere).  No reference test covers this forward:
parity unpinned against the reference; the functions below are pinned by
the closed-form checks in tests/test_oracle.py (RoPE: rotation, norm and
relative-position invariance; attention: brute-force softmax; rmsnorm).
"""
from __future__ import annotations

import numpy as np


def rmsnorm(x, w, eps):
    x = np.asarray(x, np.float64)
    return x / np.sqrt(np.mean(x * x) + eps) * np.asarray(w, np.float64)


def rope(x, pos, theta):
    """Rotate-half RoPE of one head vector x (length D) at position pos."""
    x = np.asarray(x, np.float64)
    D = x.size
    j = np.arange(D // 2)
    ang = pos * theta ** (-2.0 * j / D)
    c, s = np.cos(ang), np.sin(ang)
    a, b = x[:D // 2], x[D // 2:]
    return np.concatenate([a * c - b * s, a * s + b * c])


def attention(q, kc, vc, n_pos):
    """q [NQ][D]; kc, vc [NKV][>=n_pos][D]; softmax(q k / sqrt(D)) v over
    positions 0..n_pos-1, query head h on kv head h // (NQ / NKV)."""
    NQ, D = q.shape
    G = NQ // kc.shape[0]
    out = np.empty((NQ, D))
    for h in range(NQ):
        k = kc[h // G, :n_pos].astype(np.float64)
        v = vc[h // G, :n_pos].astype(np.float64)
        s = k @ q[h] / np.sqrt(D)
        p = np.exp(s - s.max())
        out[h] = p @ v / p.sum()
    return out


def silu_mul(g, u):
    with np.errstate(over="ignore"):   # exp(-g) = inf for g << 0 gives g / inf = -0, the limit
        return g / (1.0 + np.exp(-g)) * u


class DenseOracle:
    """Dequantises the model's weights once (oracle.dequant_rows, bit-exact to
    the reference's decoders) and runs decode steps in float64 with its own
    fp64 KV cache."""

    def __init__(self, oracle, cfg, host):
        """host["layers"][l] holds wqkv (or wq, wk, wv), wo, wgu (or wgate,
        wup), wdown and the norms; an optional qt_<name> gives that matrix's
        qtype (default cfg.qtype_layers)."""
        c = self.cfg = cfg
        D, NQ, NKV = c.head_dim, c.n_heads, c.n_kv_heads
        deq = lambda W, qt, M, K: oracle.dequant_rows(W, qt, M, K).astype(np.float64)
        QR = (NQ + 2 * NKV) * D
        self.layers = []
        for t in host["layers"]:
            qt = lambda name: t.get("qt_" + name, c.qtype_layers)
            if "wqkv" in t:
                wqkv = deq(t["wqkv"], qt("wqkv"), QR, c.hidden)
            else:
                wqkv = np.concatenate([deq(t["wq"], qt("wq"), NQ * D, c.hidden),
                                       deq(t["wk"], qt("wk"), NKV * D, c.hidden),
                                       deq(t["wv"], qt("wv"), NKV * D, c.hidden)])
            if "wgu" in t:
                wgu = deq(t["wgu"], qt("wgu"), 2 * c.ffn, c.hidden)
            else:
                wgu = np.concatenate([deq(t["wgate"], qt("wgate"), c.ffn, c.hidden),
                                      deq(t["wup"], qt("wup"), c.ffn, c.hidden)])
            self.layers.append({
                "attn_norm": t["attn_norm"], "q_norm": t["q_norm"], "k_norm": t["k_norm"],
                "ffn_norm": t["ffn_norm"], "wqkv": wqkv,
                "wo": deq(t["wo"], qt("wo"), c.hidden, NQ * D),
                "wgu": wgu,
                "wdown": deq(t["wdown"], qt("wdown"), c.hidden, c.ffn)})
        self.lm = deq(host["lm_head"], c.qtype_embd, c.vocab, c.hidden)
        self.output_norm = host["output_norm"]
        shape = (c.n_layers, c.n_kv_heads, c.max_ctx, c.head_dim)
        self.kc = np.zeros(shape)
        self.vc = np.zeros(shape)

    def decode(self, token, pos):
        c = self.cfg
        D, NQ, NKV = c.head_dim, c.n_heads, c.n_kv_heads
        x = self.lm[token].copy()           # tied embeddings: tok_embd is lm_head
        for l, L in enumerate(self.layers):
            h = rmsnorm(x, L["attn_norm"], c.norm_eps)
            qkv = L["wqkv"] @ h
            q = qkv[:NQ * D].reshape(NQ, D)
            k = qkv[NQ * D:(NQ + NKV) * D].reshape(NKV, D)
            v = qkv[(NQ + NKV) * D:].reshape(NKV, D)
            q = np.stack([rope(rmsnorm(q[i], L["q_norm"], c.norm_eps), pos, c.rope_theta) for i in range(NQ)])
            k = np.stack([rope(rmsnorm(k[i], L["k_norm"], c.norm_eps), pos, c.rope_theta) for i in range(NKV)])
            self.kc[l, :, pos] = k
            self.vc[l, :, pos] = v
            att = attention(q, self.kc[l], self.vc[l], pos + 1)
            x = x + L["wo"] @ att.reshape(-1)
            h = rmsnorm(x, L["ffn_norm"], c.norm_eps)
            gu = L["wgu"] @ h
            x = x + L["wdown"] @ silu_mul(gu[:c.ffn], gu[c.ffn:])
        return self.lm @ rmsnorm(x, self.output_norm, c.norm_eps)


def decode_layer_major(oracle, cfg, host, tokens):
    """Logits of decode steps token[i] at position i (i = 0, 1, ...) from an
    empty cache, computed layer by layer: a layer's matrices are dequantised
    (float64) once, applied to every position in order, and dropped, so a
    full-size model never holds more than one layer's weights.  The same
    arithmetic as DenseOracle.decode (layer l of position i reads only layer
    l's K/V of positions <= i)."""
    c = cfg
    D, NQ, NKV = c.head_dim, c.n_heads, c.n_kv_heads
    QR = (NQ + 2 * NKV) * D
    deq = lambda W, qt, M, K: oracle.dequant_rows(W, qt, M, K).astype(np.float64)
    lm_q = host["lm_head"]
    row_bytes = lm_q.size // c.vocab
    xs = [oracle.dequant_rows(lm_q.reshape(c.vocab, row_bytes)[t], c.qtype_embd, 1, c.hidden)[0].astype(np.float64)
          for t in tokens]
    n = len(tokens)
    for t in host["layers"]:
        qt = c.qtype_layers
        wqkv = deq(t["wqkv"], qt, QR, c.hidden)
        kc = np.zeros((NKV, n, D))
        vc = np.zeros((NKV, n, D))
        hs = []
        for i in range(n):
            qkv = wqkv @ rmsnorm(xs[i], t["attn_norm"], c.norm_eps)
            q = qkv[:NQ * D].reshape(NQ, D)
            k = qkv[NQ * D:(NQ + NKV) * D].reshape(NKV, D)
            v = qkv[(NQ + NKV) * D:].reshape(NKV, D)
            q = np.stack([rope(rmsnorm(q[h], t["q_norm"], c.norm_eps), i, c.rope_theta) for h in range(NQ)])
            kc[:, i] = np.stack([rope(rmsnorm(k[h], t["k_norm"], c.norm_eps), i, c.rope_theta) for h in range(NKV)])
            vc[:, i] = v
            hs.append(attention(q, kc, vc, i + 1).reshape(-1))
        del wqkv
        wo = deq(t["wo"], qt, c.hidden, NQ * D)
        xs = [xs[i] + wo @ hs[i] for i in range(n)]
        del wo
        wgu = deq(t["wgu"], qt, 2 * c.ffn, c.hidden)
        gus = [wgu @ rmsnorm(x, t["ffn_norm"], c.norm_eps) for x in xs]
        del wgu
        wdown = deq(t["wdown"], qt, c.hidden, c.ffn)
        xs = [x + wdown @ silu_mul(gu[:c.ffn], gu[c.ffn:]) for x, gu in zip(xs, gus)]
        del wdown
    lm = deq(lm_q, c.qtype_embd, c.vocab, c.hidden)
    return [lm @ rmsnorm(x, host["output_norm"], c.norm_eps) for x in xs]
