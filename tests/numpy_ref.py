"""Independent float64 numpy model of one Qwen3 verify step (tests only).

Written from the Qwen3 definition (RMSNorm, per-head q/k RMSNorm, NEOX RoPE with
theta_i = pos * base^(-2i/d), GQA with kv head h // (n_heads/n_kv_heads), causal
softmax attention scaled by 1/sqrt(d), SwiGLU) in float64 over the dequantized
q8_0 weights. Activations are converted to q8_0 per 32-block before every matmul
(the reference's ggml CPU path does this for q8_0 weights); everything else is
float64, so agreement with the oracle checks the composition of the ops, not
their float rounding.
"""
import numpy as np


def f16_round(x):
    return np.asarray(x, np.float32).astype(np.float16).astype(np.float64)


def q8_act(x):
    """q8_0 activation conversion: d = amax/127 (f16), codes = rint(x*127/amax)."""
    x = np.asarray(x, np.float32)
    shp = x.shape
    b = x.reshape(-1, 32)
    amax = np.abs(b).max(axis=1, keepdims=True)
    with np.errstate(divide="ignore"):
        idv = np.where(amax > 0, np.float32(127.0) / amax, np.float32(0.0)).astype(np.float32)
    codes = np.rint((b * idv).astype(np.float32))
    d = f16_round((amax / np.float32(127.0)).astype(np.float32))
    return (codes * d).reshape(shp)


def rms(x, w, eps):
    x = np.asarray(x, np.float64)
    return x / np.sqrt((x * x).mean(axis=-1, keepdims=True) + eps) * w


def rope(x, pos, base):
    d = x.shape[-1]
    half = d // 2
    i = np.arange(half)
    theta = pos * base ** (-2.0 * i / d)
    c, s = np.cos(theta), np.sin(theta)
    x0, x1 = x[..., :half], x[..., half:]
    return np.concatenate([x0 * c - x1 * s, x0 * s + x1 * c], axis=-1)


class NumpyQwen3:
    def __init__(self, model, layer_weights):
        """layer_weights: list of dicts of float64 matrices (N x K) and gains."""
        self.hp = model.hp
        self.L = layer_weights
        self.k = [[] for _ in layer_weights]
        self.v = [[] for _ in layer_weights]

    def step(self, x):
        """x: T x hidden embeddings; returns the T x hidden hidden before the output norm."""
        hp = self.hp
        D, NH, NKV = hp.head_dim, hp.n_heads, hp.n_kv_heads
        grp = NH // NKV
        x = np.asarray(x, np.float64)
        T = x.shape[0]
        for l, w in enumerate(self.L):
            past = len(self.k[l])
            xn = q8_act(rms(x, w["attn_norm"], hp.rms_eps))
            q = (xn @ w["attn_q"].T).reshape(T, NH, D)
            k = (xn @ w["attn_k"].T).reshape(T, NKV, D)
            v = (xn @ w["attn_v"].T).reshape(T, NKV, D)
            q = rms(q, w["attn_q_norm"], hp.rms_eps)
            k = rms(k, w["attn_k_norm"], hp.rms_eps)
            for t in range(T):
                q[t] = rope(q[t], past + t, hp.rope_base)
                k[t] = rope(k[t], past + t, hp.rope_base)
                self.k[l].append(k[t])
                self.v[l].append(v[t])
            K = np.stack(self.k[l])  # kv x NKV x D
            V = np.stack(self.v[l])
            o = np.zeros((T, NH, D))
            for h in range(NH):
                g = h // grp
                s = q[:, h, :] @ K[:, g, :].T / np.sqrt(D)  # T x kv
                for t in range(T):
                    s[t, past + t + 1:] = -np.inf
                s = s - s.max(axis=1, keepdims=True)
                p = np.exp(s)
                p /= p.sum(axis=1, keepdims=True)
                o[:, h, :] = p @ V[:, g, :]
            o = q8_act(o.reshape(T, NH * D))
            x = x + o @ w["attn_o"].T
            hn = q8_act(rms(x, w["ffn_norm"], hp.rms_eps))
            g_ = hn @ w["ffn_gate"].T
            u = hn @ w["ffn_up"].T
            a = q8_act(g_ / (1.0 + np.exp(-g_)) * u)
            x = x + a @ w["ffn_down"].T
        return x


def layer_weights(model):
    """Dequantized float64 weights of every layer of a SynthModel."""
    import ctypes
    import mtg
    hp = model.hp
    H, D, F = hp.hidden, hp.head_dim, hp.intermediate
    QN, KN = hp.n_heads * D, hp.n_kv_heads * D
    out = []
    for l in range(hp.n_layers):
        t = model.desc.contents.layers[l]
        def mat(p, k, n):
            return model.dequant_rows(p, k, range(n)).astype(np.float64)
        def gain(p, n):
            return np.frombuffer(ctypes.string_at(p, 4 * n), np.float32).astype(np.float64)
        out.append(dict(
            attn_q=mat(t.attn_q, H, QN), attn_k=mat(t.attn_k, H, KN), attn_v=mat(t.attn_v, H, KN),
            attn_o=mat(t.attn_o, QN, H), ffn_gate=mat(t.ffn_gate, H, F), ffn_up=mat(t.ffn_up, H, F),
            ffn_down=mat(t.ffn_down, F, H), attn_norm=gain(t.attn_norm, H), ffn_norm=gain(t.ffn_norm, H),
            attn_q_norm=gain(t.attn_q_norm, D), attn_k_norm=gain(t.attn_k_norm, D)))
    return out
