"""Independent float64 statement of mdma's Llama forward, for pinning the
oracle's composition (test infrastructure).

Written from the reference's layer loop, /root/reference/src/model/arch/llama.rs:158-246
(rmsnorm, or add + rmsnorm of the residual stream, before attention; QKV;
RoPE of q and k with the rotated k and the plain v cached; causal GQA
attention; o projection; add + rmsnorm before the FFN; gate/up with SiLU;
down projection; a final add + rmsnorm), and from the CPU backend's per-op
semantics (src/backend/cpu.rs: rmsnorm :388-402 with 1/sqrt(mean + eps) per
row; apply_rope :68-84, interleaved pairs, freq = theta^(-2i/hd); attention
:530-590 with scale 1/sqrt(hd) and a max-shifted softmax; silu_mul
:447-458). Model::prefill and forward (src/model.rs:326-468) take the head on
the last row. Every value is float64 and the weights are the exact block
values of tests/npq.py; nothing here calls oracle/.
"""
from __future__ import annotations

import numpy as np

import npq


class LlamaF64:
    def __init__(self, reader):
        md = reader.metadata
        a = md["general.architecture"]
        self.E = md[f"{a}.embedding_length"]
        self.L = md[f"{a}.block_count"]
        self.H = md[f"{a}.attention.head_count"]
        self.KVH = md.get(f"{a}.attention.head_count_kv", self.H)
        self.hd = self.E // self.H
        self.eps = float(md[f"{a}.attention.layer_norm_rms_epsilon"])
        self.theta = float(md.get(f"{a}.rope.freq_base", 10000.0))
        self.r = reader
        self._cache = {}

    def w(self, name):
        if name not in self._cache:
            t = self.r.tensors[name]
            raw = self.r.bytes_of(name)
            if len(t.shape) == 1:
                self._cache[name] = npq.dequantize(t.dtype, raw, 1, t.shape[0])[0]
            else:
                self._cache[name] = npq.dequantize(t.dtype, raw, t.shape[0], t.shape[1])
        return self._cache[name]

    def rmsnorm(self, x, g):
        ms = np.mean(x * x, axis=-1, keepdims=True)
        return x / np.sqrt(ms + self.eps) * g

    def rope(self, v, positions, n_heads):
        """v [T, n_heads*hd]; pair (2i, 2i+1) of each head rotated by pos*freq_i."""
        hd, half = self.hd, self.hd // 2
        freq = self.theta ** (-2.0 * np.arange(half) / hd)
        ang = np.asarray(positions, np.float64)[:, None] * freq[None, :]
        c, s = np.cos(ang)[:, None, :], np.sin(ang)[:, None, :]
        h = v.reshape(v.shape[0], n_heads, half, 2)
        x0, x1 = h[..., 0], h[..., 1]
        out = np.stack([x0 * c - x1 * s, x0 * s + x1 * c], axis=-1)
        return out.reshape(v.shape)

    def attention(self, q, kc, vc, n_keys):
        """q [T, H*hd] for the last T of n_keys positions; kc/vc [n_keys, KVH*hd]."""
        T, hd, G = q.shape[0], self.hd, self.H // self.KVH
        o = np.zeros_like(q)
        for t in range(T):
            vis = n_keys - T + t + 1
            for h in range(self.H):
                kv = h // G
                qv = q[t, h * hd:(h + 1) * hd]
                K = kc[:vis, kv * hd:(kv + 1) * hd]
                V = vc[:vis, kv * hd:(kv + 1) * hd]
                sc = K @ qv / np.sqrt(hd)
                p = np.exp(sc - sc.max())
                o[t, h * hd:(h + 1) * hd] = (p / p.sum()) @ V
        return o

    def forward_all(self, tokens, n_prompt: int):
        """Logits of every step of a token sequence: the prompt's last row,
        then each later token fed one at a time (teacher forcing).
        Returns [len(tokens) - n_prompt + 1, vocab]."""
        E, L, hd = self.E, self.L, self.hd
        kvw = self.KVH * hd
        n = len(tokens)
        kc = [np.zeros((n, kvw)) for _ in range(L)]
        vc = [np.zeros((n, kvw)) for _ in range(L)]
        emb = self.w("token_embd.weight")
        out = []
        chunks = [(0, n_prompt)] + [(p, p + 1) for p in range(n_prompt, n)]
        for p0, p1 in chunks:
            x = emb[np.asarray(tokens[p0:p1])]
            proj = None
            for i in range(L):
                pre = f"blk.{i}."
                if proj is not None:
                    x = x + proj
                h = self.rmsnorm(x, self.w(pre + "attn_norm.weight"))
                q = h @ self.w(pre + "attn_q.weight").T
                k = h @ self.w(pre + "attn_k.weight").T
                v = h @ self.w(pre + "attn_v.weight").T
                pos = np.arange(p0, p1)
                q, k = self.rope(q, pos, self.H), self.rope(k, pos, self.KVH)
                kc[i][p0:p1], vc[i][p0:p1] = k, v
                a = self.attention(q, kc[i], vc[i], p1)
                x = x + a @ self.w(pre + "attn_output.weight").T
                h = self.rmsnorm(x, self.w(pre + "ffn_norm.weight"))
                g = h @ self.w(pre + "ffn_gate.weight").T
                u = h @ self.w(pre + "ffn_up.weight").T
                proj = (g / (1.0 + np.exp(-g)) * u) @ self.w(pre + "ffn_down.weight").T
            x = x + proj
            hN = self.rmsnorm(x[-1:], self.w("output_norm.weight"))
            out.append((hN @ self.w("output.weight").T)[0])
            if p1 == n:
                break
        return np.stack(out)
