"""A Llama forward made only of trait-level calls on the C ABI, and a graph
decoder over it: the shape of the reference's Model::forward_device
(/root/reference/src/model.rs:355-387 with Llama::run_layers,
src/model/arch/llama.rs:158-246, and KvCache::rope_write,
src/kv_cache.rs:212-244) and of HipDecoder (src/backend/rocm/graph.rs:
105-262), which a Rust Gfx950Backend::decoder(model, kv, ws) would run over
mdma's own Model / KvCache / Workspace buffers. Test support: the weights are
uploaded through the trait-shaped upload_weight (raw GGUF bytes, repacked on
the device at first use)."""
import numpy as np

from mdma_amd import gguf
from mdma_amd.backend import AttnSpec, KvView, QWeight, RopeSpec


class TraitLlama:
    def __init__(self, be, path: str, capacity: int, rows: int):
        r = gguf.Reader(path)
        md = r.metadata
        self.be = be
        self.E = int(md["llama.embedding_length"])
        self.H = int(md["llama.attention.head_count"])
        self.KVH = int(md["llama.attention.head_count_kv"])
        self.F = int(md["llama.feed_forward_length"])
        self.L = int(md["llama.block_count"])
        self.eps = float(md["llama.attention.layer_norm_rms_epsilon"])
        self.theta = float(md["llama.rope.freq_base"])
        self.hd = self.E // self.H
        self.V = r.tensors["output.weight"].shape[0]
        self.cap = capacity

        def w(name):
            t = r.tensors[name]
            return QWeight(t.dtype, tuple(t.shape), be.upload_weight_bytes(r.bytes_of(name)))

        def n(name):
            return be.f32_buf(np.frombuffer(r.bytes_of(name), np.float32))

        self.te, self.out, self.out_norm = w("token_embd.weight"), w("output.weight"), n("output_norm.weight")
        self.layers = []
        for i in range(self.L):
            p = f"blk.{i}."
            self.layers.append({k: (n(p + k + ".weight") if k.endswith("norm") else w(p + k + ".weight"))
                                for k in ("attn_norm", "attn_q", "attn_k", "attn_v", "attn_output", "ffn_norm",
                                          "ffn_gate", "ffn_up", "ffn_down")})
        kvw = self.KVH * self.hd
        self.kc = [be.alloc(capacity * kvw * 2) for _ in range(self.L)]
        self.vc = [be.alloc(capacity * kvw * 2) for _ in range(self.L)]
        E, F = self.E, self.F
        # Workspace (src/model/memory.rs:39-63): per buffer its width per token row.
        self.width = {"x": E, "x_alt": E, "normed": E, "proj": E, "q": self.H * self.hd, "k": kvw, "v": kvw,
                      "attn_out": self.H * self.hd, "gate": F, "up": F, "act": F}
        self.ws = {k: be.alloc(rows * n_ * 4) for k, n_ in self.width.items()}
        self.logits = be.alloc(self.V * 4)

    def run(self, tokens, pos: int):
        """Llama::run + the head on the last row: embed, the layers, the output norm."""
        be, ws, T = self.be, self.ws, len(tokens)
        kvw = self.KVH * self.hd
        # Views of T token rows: the ops infer T from the buffers' lengths.
        v = {k: be.view(b, 0, T * self.width[k] * 4) for k, b in ws.items()}
        be.embed(self.te, np.asarray(tokens, np.uint32), v["x"])
        rope, att = RopeSpec(self.hd, self.theta), AttnSpec(self.hd, self.H, self.KVH)
        x, xa = v["x"], v["x_alt"]
        for i, L in enumerate(self.layers):
            if i == 0:
                be.rmsnorm(L["attn_norm"], x, v["normed"], self.eps)
            else:
                be.add_rmsnorm(L["attn_norm"], x, v["proj"], xa, v["normed"], self.eps)
                x, xa = xa, x
            be.qmatmul_qkv(L["attn_q"], L["attn_k"], L["attn_v"], v["normed"], v["q"], v["k"], v["v"])
            be.rope_kv_write(v["q"], v["k"], v["v"], self.kc[i], self.vc[i], pos * kvw, pos, T, rope, T * kvw)
            be.attn(v["q"], KvView(self.kc[i], self.vc[i], pos + T), att, v["attn_out"])
            be.qmatmul(L["attn_output"], v["attn_out"], v["proj"])
            be.add_rmsnorm(L["ffn_norm"], x, v["proj"], xa, v["normed"], self.eps)
            x, xa = xa, x
            be.ffn_gate_up(L["ffn_gate"], L["ffn_up"], v["normed"], v["gate"], v["up"], v["act"])
            be.qmatmul(L["ffn_down"], v["act"], v["proj"])
        be.add_rmsnorm(self.out_norm, x, v["proj"], xa, v["normed"], self.eps)
        last = be.view(v["normed"], (T - 1) * self.E * 4, self.E * 4)
        be.qmatmul(self.out, last, self.logits)
        for b in list(v.values()) + [last]:
            b.close()

    def forward(self, token: int, pos: int) -> np.ndarray:
        """Model::forward: one decode step, eagerly; the logits."""
        self.run([token], pos)
        return self.be.download_f32(self.logits)


class TraitDecoder:
    """HipDecoder over TraitLlama: the decode step captured once with the
    replay parameters set, then replayed with [token, position] written to
    device memory before each launch."""

    def __init__(self, model: TraitLlama):
        self.m = model
        self.params = model.be.alloc(8)
        self.graph = None
        self.replayed = False

    def forward(self, token: int, pos: int) -> np.ndarray:
        be = self.m.be
        be.upload(self.params, 0, np.array([token, pos], np.uint32))
        self.replayed = False
        if self.graph is not None:
            try:
                self.graph.launch()
                self.replayed = True
            except Exception:  # the context replaced a buffer the graph captured
                self.graph.close()
                self.graph = None
        if not self.replayed:
            be.set_replay_params(self.params, self.m.cap)
            try:
                self.m.run([0], 0)  # eager, reading token and position from params: sizes every buffer
                self.graph = be.capture(lambda: self.m.run([0], 0))
            finally:
                be.set_replay_params(None)
        return be.download_f32(self.m.logits)

    def close(self):
        if self.graph is not None:
            self.graph.close()
        self.params.close()
