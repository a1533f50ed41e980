"""CPU restatement of the reference's BitLlama inference step, composed from the
oracle's restated ops (bitlinear_oracle.c, bitllama_oracle.c).

TEST INFRASTRUCTURE ONLY: imported by tests/ and __graft_entry__.smoke() as the
checker of bitlinear.model.BitLlamaHip.  The product package never imports it.

Follows (imonoonoko/Bit-TTT-Engine, crates/rust_engine/src):
  BitLlama::forward_one       model/llama.rs:201-271
  BitLlamaBlock::forward      model/block.rs:90-138
  BitAttention::forward       layers/attention.rs:149-224 (one query per step)
  QuantizedKVCache::append    layers/kv_cache.rs:49-119
  SwiGLU::forward             layers/swiglu.rs:29-35
with every linear a W1.58-A8 BitLinear (orc_forward_i8) and RMSNorm as
orc_rmsnorm.  Token by token, as the reference's stream_completion feeds the
prompt (llama.rs:489-493).
"""
import numpy as np

from . import oracle as orc


class OracleLlama:
    """cfg: an object with hidden, n_layers, n_heads, n_kv_heads, head_dim,
    intermediate, vocab, rope_theta, max_seq, eps.  w: host weights
      embed [vocab, hidden] f32, norm_f [hidden] f32,
      lm_head (bytes, scale) -- or a dense [vocab, hidden] f32 array / uint16 array
      of bf16 bits (the reference's candle_nn::Linear), layers: [{norm1, norm2, q,
      k, v, o, gate, up, down}]
    with the linears as (packed bytes uint8, scale) pairs.  mode "i8": every
    BitLinear in W1.58-A8; "f32_ref": in the reference's own fp32 arithmetic
    (BitLinearCpu, cpu.rs:17-127), the decoder the reference runs on a CPU."""

    def __init__(self, cfg, w, mode="i8"):
        assert mode in ("i8", "f32_ref")
        self.cfg, self.w, self.mode = cfg, w, mode
        c = cfg
        self.cos, self.sin = orc.rope_table(c.rope_theta, c.head_dim, c.max_seq)
        self.caches = [dict(kq=np.zeros((c.n_kv_heads, c.max_seq, c.head_dim), np.uint8),
                            ks=np.zeros((c.n_kv_heads, c.max_seq), np.float32),
                            vq=np.zeros((c.n_kv_heads, c.max_seq, c.head_dim), np.uint8),
                            vs=np.zeros((c.n_kv_heads, c.max_seq), np.float32)) for _ in range(c.n_layers)]
        self.pos = 0

    def _lin(self, x, pk, n):
        if self.mode == "f32_ref":  # BitLinearCpu::forward's fp32 order (cpu.rs:17-127)
            return orc.forward_f32(x, pk[0], n, np.float32(pk[1]))
        return orc.forward_i8(x, pk[0], n, pk[1])[0]

    def forward_one(self, token):
        c, w = self.cfg, self.w
        pos = self.pos
        hd, nh, nkv = c.head_dim, c.n_heads, c.n_kv_heads
        h = np.ascontiguousarray(w["embed"][int(token)][None, :], np.float32)
        for li, L in enumerate(w["layers"]):
            xn = orc.rmsnorm(h, L["norm1"], c.eps)
            q = self._lin(xn, L["q"], nh * hd)[0]
            k = self._lin(xn, L["k"], nkv * hd)[0]
            v = self._lin(xn, L["v"], nkv * hd)[0]
            q = orc.rope_apply(q.reshape(nh, hd), self.cos[pos], self.sin[pos]).reshape(-1)
            k = orc.rope_apply(k.reshape(nkv, hd), self.cos[pos], self.sin[pos])
            kq, ks = orc.q8_quant(k)
            vq, vs = orc.q8_quant(v.reshape(nkv, hd))
            C = self.caches[li]
            C["kq"][:, pos], C["ks"][:, pos] = kq, ks
            C["vq"][:, pos], C["vs"][:, pos] = vq, vs
            a = orc.attn_decode(q, C["kq"], C["ks"], C["vq"], C["vs"], nh, pos + 1)
            o = self._lin(a[None, :], L["o"], c.hidden)
            h = (h + o).astype(np.float32)
            xn2 = orc.rmsnorm(h, L["norm2"], c.eps)
            g = self._lin(xn2, L["gate"], c.intermediate)
            u = self._lin(xn2, L["up"], c.intermediate)
            d = self._lin(orc.swiglu(g, u), L["down"], c.hidden)
            h = (h + d).astype(np.float32)
        xf = orc.rmsnorm(h, w["norm_f"], c.eps)
        head = w["lm_head"]
        if isinstance(head, np.ndarray):  # dense f32 / bf16-bits [vocab, hidden] (llama.rs:129-141)
            logits = orc.dense_linear(xf, head)[0]
        else:
            logits = self._lin(xf, head, c.vocab)[0]
        self.pos += 1
        return logits

    def generate(self, prompt, max_tokens):
        """Prefill token by token, then greedy decode starting from the prompt's
        last logits; returns the generated ids."""
        logits = None
        for t in prompt:
            logits = self.forward_one(t)
        out = []
        tok = orc.argmax(logits)
        out.append(tok)
        while len(out) < max_tokens:
            tok = orc.argmax(self.forward_one(tok))
            out.append(tok)
        return np.array(out, dtype=np.int32)
