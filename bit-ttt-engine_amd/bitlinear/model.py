"""A Llama-shaped ternary decoder on the C ABI: the host side of the reference's
BitLlama inference path with every BitLinear and the ops around it on the GPU.

Reference (imonoonoko/Bit-TTT-Engine, crates/rust_engine/src):
  BitLlama::forward_one            model/llama.rs:201-271   (embedding, blocks, norm, lm_head)
  BitLlamaBlock::forward           model/block.rs:90-138    (norm1, attention, residual, norm2, MLP, residual)
  BitAttention::forward            layers/attention.rs:149-224 (q/k/v, RoPE, Q8 cache, softmax, o_proj)
  QuantizedKVCache                 layers/kv_cache.rs:14-128
  SwiGLU::forward                  layers/swiglu.rs:29-35
  Llama::stream_completion         model/llama.rs:471-530   (prefill, then greedy decode)

Mapping of the block onto the C ABI (one row of activations per token, f32 between ops):
  x = h + mlp_out(l-1); q,k,v = BitLinear(RMSNorm1(x))   btl_add_rmsnorm_linear_group
  RoPE(q, k); cache.append(k, v);
  attn = softmax(q k^T / sqrt(d)) v                      btl_rope_append_attention
  o = BitLinear_o(attn)                                  btl_linear_group
  x' = x + o; hs = silu(W1 RMSNorm2(x')) * W3 RMSNorm2(x')  btl_add_rmsnorm_swiglu
  mlp_out = BitLinear_down(hs)                           btl_linear_group
(many rows: gate and up through btl_add_rmsnorm_linear_group, then
mlp_out = BitLinear_down(silu(gate) * up) through btl_swiglu_linear_group, the
SwiGLU in the down call's quantiser; same bits), and after the last block logits = lm_head(RMSNorm_f(x' + mlp_out)) in one more
btl_add_rmsnorm_linear_group.  The residual stream alternates between two
buffers (each add writes the other one).  A one-token step moves the two adds
into the epilogues of o and down (x' = x + o and x + mlp_out through
btl_linear_residual), so the kernels of q|k|v and gate|up apply only the
RMSNorm, in their quantising waves; the gate/up kernel writes silu(gate) * up
from its epilogue.  Every linear of the blocks is a BitLinear (W1.58-A8); the
lm_head is either a BitLinear too (one launch with the final norm) or, as in the
reference, a dense linear (llama.rs:129-141: btl_add_rmsnorm, then
btl_dense_linear over f32 or bf16 weights).

Deliberate differences from the reference, all on the host side:
  * the prompt is prefilled as one batch of rows (the reference feeds it token by
    token through forward_one, llama.rs:489-493); every op is row-independent or
    causal, so the state and logits are the same bits as token-by-token steps
    (a GPU test checks this);
  * the first decode step feeds the token chosen from the prompt's last logits
    (the reference feeds the last prompt token a second time, llama.rs:496-499);
  * the TTT layer variant and sampling with temperature are not built.
"""
import ctypes

import numpy as np
import torch

from ._lib import BTL_ACT_F32_REF, BTL_F32, BTL_BF16, BtlKvQ8, BtlPacked, check, lib
from .packed import PackedTensor

RMS_NORM_EPS = 1e-5  # block.rs:10


class LlamaConfig:
    """The shape fields of BitLlamaConfig (model/config.rs) the decoder needs."""

    def __init__(self, hidden, n_layers, n_heads, n_kv_heads, intermediate, vocab, rope_theta=500000.0,
                 max_seq=1024, eps=RMS_NORM_EPS):
        self.hidden = hidden
        self.n_layers = n_layers
        self.n_heads = n_heads
        self.n_kv_heads = n_kv_heads
        self.head_dim = hidden // n_heads
        self.intermediate = intermediate
        self.vocab = vocab
        self.rope_theta = rope_theta
        self.max_seq = max_seq
        self.eps = eps

    @staticmethod
    def llama3_8b(max_seq=1024):
        """models/Meta-Llama-3-8B/config.json shapes."""
        return LlamaConfig(4096, 32, 32, 8, 14336, 128256, 500000.0, max_seq)


class KVCacheQ8:
    """QuantizedKVCache (kv_cache.rs:14-128) of one layer, allocated for max_seq rows."""

    def __init__(self, n_kv_heads, max_seq, head_dim, device):
        self.k = torch.zeros((n_kv_heads, max_seq, head_dim), dtype=torch.uint8, device=device)
        self.v = torch.zeros_like(self.k)
        self.k_scale = torch.zeros((n_kv_heads, max_seq), dtype=torch.float32, device=device)
        self.v_scale = torch.zeros_like(self.k_scale)
        self.c = BtlKvQ8(self.k.data_ptr(), self.v.data_ptr(), self.k_scale.data_ptr(), self.v_scale.data_ptr(),
                         n_kv_heads, max_seq, head_dim)

    def reset(self):
        """kv_cache.rs:38-45 (rows are overwritten by the next appends)."""
        self.k.zero_()
        self.v.zero_()
        self.k_scale.zero_()
        self.v_scale.zero_()


def _arr(packed):
    cs = [p.as_c() for p in packed]
    return cs, (ctypes.POINTER(BtlPacked) * len(cs))(*[ctypes.pointer(c) for c in cs])


def _ptrs(ts):
    return (ctypes.c_void_p * len(ts))(*[t.data_ptr() for t in ts])


class BitLlamaHip:
    """BitLlama with attention blocks (ModelArch::Llama), all linears packed ternary.

    mode "i8" runs every BitLinear in W1.58-A8 with the fused decode kernels;
    mode "f32_ref" runs them in the reference's own fp32 arithmetic
    (BitLinearCpu::forward, cpu.rs:17-127, bit for bit) -- with a dense f32
    lm_head this is the decoder the reference runs on a CPU.

    weights: dict with
      "embed" [vocab, hidden] float32 or bfloat16 (GPU),
      "norm_f" [hidden] float32, "lm_head" PackedTensor [vocab, hidden] (ternary, a
      BitLinear) or a dense float32 / bfloat16 tensor [vocab, hidden] (the
      reference's candle_nn::Linear, llama.rs:129-141),
      "layers": list of dicts {"norm1", "norm2": [hidden] f32,
                               "q", "k", "v", "o", "gate", "up", "down": PackedTensor}.
    """

    def __init__(self, cfg, weights, device="cuda", max_rows=512, mode="i8"):
        if mode not in ("i8", "f32_ref"):
            raise ValueError("mode is 'i8' (W1.58-A8) or 'f32_ref' (the reference's fp32 BitLinear)")
        self.mode = mode
        self.cfg = cfg
        self.dev = torch.device(device)
        self.w = weights
        self.max_rows = max_rows
        c = cfg
        f32 = dict(dtype=torch.float32, device=self.dev)
        M = max_rows
        self.h = torch.zeros((M, c.hidden), **f32)   # residual stream, alternating with h2
        self.h2 = torch.zeros((M, c.hidden), **f32)
        self.q = torch.zeros((M, c.n_heads * c.head_dim), **f32)
        self.k = torch.zeros((M, c.n_kv_heads * c.head_dim), **f32)
        self.v = torch.zeros((M, c.n_kv_heads * c.head_dim), **f32)
        self.attn = torch.zeros((M, c.n_heads * c.head_dim), **f32)
        self.o = torch.zeros((M, c.hidden), **f32)
        self.hs = torch.zeros((M, c.intermediate), **f32)  # silu(gate) * up
        self.down = torch.zeros((M, c.hidden), **f32)
        if mode == "f32_ref":
            self.xn = torch.zeros((M, c.hidden), **f32)         # the normed rows
        if mode == "f32_ref" or M > 1:
            # gate and up of many rows (SwiGLU then runs in the down call's quantiser)
            self.gate = torch.zeros((M, c.intermediate), **f32)
            self.up = torch.zeros((M, c.intermediate), **f32)
        self.logits = torch.zeros((1, c.vocab), **f32)
        self.ids = torch.zeros((M,), dtype=torch.int32, device=self.dev)
        self.next_id = torch.zeros((1,), dtype=torch.int32, device=self.dev)
        self.d_pos = torch.zeros((1,), dtype=torch.int32, device=self.dev)
        self.log = torch.zeros((c.max_seq + 1,), dtype=torch.int32, device=self.dev)
        cos = np.zeros((c.max_seq, c.head_dim // 2), np.float32)
        sin = np.zeros_like(cos)
        check(lib.btl_rope_table(float(c.rope_theta), c.head_dim, c.max_seq, cos.ctypes.data, sin.ctypes.data))
        self.rope_cos = torch.from_numpy(cos).to(self.dev)
        self.rope_sin = torch.from_numpy(sin).to(self.dev)
        self.caches = [KVCacheQ8(c.n_kv_heads, c.max_seq, c.head_dim, self.dev) for _ in range(c.n_layers)]
        emb = weights["embed"]
        self.emb_dtype = BTL_BF16 if emb.dtype == torch.bfloat16 else BTL_F32
        # pre-bound C arguments (pointers resolved once)
        self._layers = []
        for L in weights["layers"]:
            qkv_c, qkv = _arr([L["q"], L["k"], L["v"]])
            o_c, o = _arr([L["o"]])
            gate_c, up_c = L["gate"].as_c(), L["up"].as_c()
            d_c, d = _arr([L["down"]])
            gu_c, gu = _arr([L["gate"], L["up"]])
            self._layers.append(dict(keep=(qkv_c, o_c, d_c, gu_c), qkv=qkv, o=o, down=d, gu=gu,
                                     o_w=ctypes.byref(o_c[0]),
                                     down_w=ctypes.byref(d_c[0]),
                                     gate=ctypes.byref(gate_c), up=ctypes.byref(up_c), gate_c=gate_c, up_c=up_c,
                                     n1=L["norm1"].data_ptr(), n2=L["norm2"].data_ptr()))
        head = weights["lm_head"]
        self.dense_head = isinstance(head, torch.Tensor)
        if self.dense_head:
            if head.dtype not in (torch.float32, torch.bfloat16) or tuple(head.shape) != (c.vocab, c.hidden) \
                    or not head.is_contiguous():
                raise ValueError("dense lm_head: a contiguous float32 / bfloat16 [vocab, hidden] tensor")
            self._head_dt = BTL_BF16 if head.dtype == torch.bfloat16 else BTL_F32
            self.xf = torch.zeros((1, c.hidden), **f32)  # RMSNorm_f of the last row
        else:
            self._head_c, self._head = _arr([head])
        self._y_qkv = _ptrs([self.q, self.k, self.v])
        self._y_o = _ptrs([self.o])
        self._y_down = _ptrs([self.down])
        self._y_logits = _ptrs([self.logits])
        if mode == "f32_ref" or M > 1:
            self._y_gu = _ptrs([self.gate, self.up])
        # the model's own workspace, sized for every call it makes, so captured
        # steps never depend on the library's shared workspace
        I8 = 1
        kvd, qd = c.n_kv_heads * c.head_dim, c.n_heads * c.head_dim
        need = max(lib.btl_workspace_bytes(M, qd + 2 * kvd, c.hidden, I8),
                   lib.btl_workspace_bytes(M, c.hidden, qd, I8),
                   lib.btl_add_rmsnorm_swiglu_workspace_bytes(M, c.intermediate, c.hidden),
                   lib.btl_workspace_bytes(M, 2 * c.intermediate, c.hidden, I8),
                   lib.btl_workspace_bytes(M, c.hidden, c.intermediate, I8),
                   lib.btl_workspace_bytes(1, c.vocab, c.hidden, I8),
                   lib.btl_attention_workspace_bytes(M, c.n_heads, ctypes.byref(self.caches[0].c)))
        self.ws = torch.empty((need + 256,), dtype=torch.uint8, device=self.dev)
        base = self.ws.data_ptr()
        self._ws = ctypes.c_void_p((base + 255) // 256 * 256)
        self._ws_n = need
        self.pos = 0
        self.graph = None

    # ------------------------------------------------------------------ steps
    def _stream(self):
        return ctypes.c_void_p(torch.cuda.current_stream(self.dev).cuda_stream)

    def _run(self, m, pos, d_pos, ids):
        """One forward of m rows, token ids in the device int32 tensor `ids`, at
        positions pos.. (or *d_pos.. when d_pos is a device tensor); leaves the last
        row's logits in self.logits."""
        c, st = self.cfg, self._stream()
        ws, wn = self._ws, self._ws_n
        dp = ctypes.c_void_p(d_pos.data_ptr()) if d_pos is not None else None
        hid = c.hidden
        check(lib.btl_embedding(self.w["embed"].data_ptr(), self.emb_dtype, c.vocab, hid, ids.data_ptr(), m,
                                self.h.data_ptr(), st))
        if self.mode == "f32_ref":
            self._run_ref(m, pos, dp, st)
            return
        cur, nxt = self.h, self.h2  # each add writes the other buffer
        # One token: the residual adds run in the epilogues of the o and down
        # projections (btl_linear_residual), so the norms ahead of q|k|v and
        # gate|up are plain RMSNorms inside those launches.  More rows: the add
        # is fused into the next norm's transform instead.  Same bits.
        one = m == 1
        for li, L in enumerate(self._layers):
            cache = self.caches[li].c
            if li > 0 and not one:
                check(lib.btl_add_rmsnorm_linear_group(L["qkv"], self._y_qkv, 3, cur.data_ptr(), self.down.data_ptr(),
                                                       nxt.data_ptr(), L["n1"], c.eps, m, hid, BTL_F32, ws, wn, st))
                cur, nxt = nxt, cur
            else:
                check(lib.btl_add_rmsnorm_linear_group(L["qkv"], self._y_qkv, 3, cur.data_ptr(), None, None, L["n1"],
                                                       c.eps, m, hid, BTL_F32, ws, wn, st))
            check(lib.btl_rope_append_attention(self.q.data_ptr(), self.k.data_ptr(), self.v.data_ptr(), m,
                                                c.n_heads, ctypes.byref(cache), pos, dp, self.rope_cos.data_ptr(),
                                                self.rope_sin.data_ptr(), self.attn.data_ptr(), ws, wn, st))
            if one:
                check(lib.btl_linear_residual(L["o_w"], self.attn.data_ptr(), BTL_F32, m, c.n_heads * c.head_dim,
                                              cur.data_ptr(), nxt.data_ptr(), ws, wn, st))
                cur, nxt = nxt, cur
                check(lib.btl_add_rmsnorm_swiglu(L["gate"], L["up"], cur.data_ptr(), None, None, L["n2"], c.eps, m,
                                                 hid, self.hs.data_ptr(), ws, wn, st))
                check(lib.btl_linear_residual(L["down_w"], self.hs.data_ptr(), BTL_F32, m, c.intermediate,
                                              cur.data_ptr(), nxt.data_ptr(), ws, wn, st))
                cur, nxt = nxt, cur
                continue
            check(lib.btl_linear_group(L["o"], self._y_o, 1, self.attn.data_ptr(), BTL_F32, m,
                                       c.n_heads * c.head_dim, BTL_F32, ws, wn, st))
            # gate and up of the summed, normed rows, then down with SwiGLU in its
            # quantiser (the same bits as silu(gate) * up written out and quantised:
            # one elementwise pass and one row of f32 traffic fewer)
            check(lib.btl_add_rmsnorm_linear_group(L["gu"], self._y_gu, 2, cur.data_ptr(), self.o.data_ptr(),
                                                   nxt.data_ptr(), L["n2"], c.eps, m, hid, BTL_F32, ws, wn, st))
            cur, nxt = nxt, cur
            check(lib.btl_swiglu_linear_group(L["down"], self._y_down, 1, self.gate.data_ptr(), self.up.data_ptr(),
                                              BTL_F32, m, c.intermediate, BTL_F32, ws, wn, st))
        last = m - 1
        delta = None if one else self.down[last].data_ptr()
        if self.dense_head:
            # RMSNorm_f into f32, then the dense linear (llama.rs:255-265)
            check(lib.btl_add_rmsnorm(cur[last].data_ptr(), delta, None, self.w["norm_f"].data_ptr(), c.eps, 1, hid,
                                      self.xf.data_ptr(), st))
            check(lib.btl_dense_linear(self.w["lm_head"].data_ptr(), self._head_dt, c.vocab, hid, self.xf.data_ptr(),
                                       1, self.logits.data_ptr(), st))
            return
        check(lib.btl_add_rmsnorm_linear_group(self._head, self._y_logits, 1, cur[last].data_ptr(), delta, None,
                                               self.w["norm_f"].data_ptr(), c.eps, 1, hid, BTL_F32, ws, wn, st))

    def _run_ref(self, m, pos, dp, st):
        """The blocks and the head in the reference's own arithmetic: every BitLinear
        as BitLinearCpu::forward (btl_linear_group_mode, BTL_ACT_F32_REF), the
        residual adds and norms through btl_add_rmsnorm (the add of a block's output
        is done by the next norm), SwiGLU's activation through btl_swiglu.  For one
        token row with a hidden width that is a multiple of 64 up to 16384 the norms
        run inside the q|k|v and gate|up launches (btl_add_rmsnorm_linear_group_ref:
        the same bits, six launches per block instead of eight)."""
        c = self.cfg
        hid, qd = c.hidden, c.n_heads * c.head_dim
        F, R = BTL_F32, BTL_ACT_F32_REF
        cur, nxt = self.h, self.h2
        delta = None  # the block output still to be added to cur
        # one token row: the norms run inside the projections' launches (more
        # rows measured slower that way: every workgroup normalises its rows again)
        fused = m == 1 and hid % 64 == 0 and 64 <= hid <= 16384
        for li, L in enumerate(self._layers):
            if fused:
                dl = delta.data_ptr() if delta is not None else None
                ho = nxt.data_ptr() if delta is not None else None
                check(lib.btl_add_rmsnorm_linear_group_ref(L["qkv"], self._y_qkv, 3, cur.data_ptr(), dl, ho, L["n1"],
                                                           c.eps, m, hid, st))
                if delta is not None:
                    cur, nxt = nxt, cur
                check(lib.btl_rope_append_attention(self.q.data_ptr(), self.k.data_ptr(), self.v.data_ptr(), m,
                                                    c.n_heads, ctypes.byref(self.caches[li].c), pos, dp,
                                                    self.rope_cos.data_ptr(), self.rope_sin.data_ptr(),
                                                    self.attn.data_ptr(), self._ws, self._ws_n, st))
                check(lib.btl_linear_group_mode(L["o"], self._y_o, 1, self.attn.data_ptr(), F, m, qd, F, R, None, 0,
                                                st))
                check(lib.btl_add_rmsnorm_linear_group_ref(L["gu"], self._y_gu, 2, cur.data_ptr(),
                                                           self.o.data_ptr(), nxt.data_ptr(), L["n2"], c.eps, m, hid,
                                                           st))
                cur, nxt = nxt, cur
                check(lib.btl_swiglu(self.gate.data_ptr(), self.up.data_ptr(), m * c.intermediate, self.hs.data_ptr(),
                                     st))
                check(lib.btl_linear_group_mode(L["down"], self._y_down, 1, self.hs.data_ptr(), F, m, c.intermediate,
                                                F, R, None, 0, st))
                delta = self.down
                continue
            if delta is None:
                check(lib.btl_add_rmsnorm(cur.data_ptr(), None, None, L["n1"], c.eps, m, hid, self.xn.data_ptr(), st))
            else:
                check(lib.btl_add_rmsnorm(cur.data_ptr(), delta.data_ptr(), nxt.data_ptr(), L["n1"], c.eps, m, hid,
                                          self.xn.data_ptr(), st))
                cur, nxt = nxt, cur
            check(lib.btl_linear_group_mode(L["qkv"], self._y_qkv, 3, self.xn.data_ptr(), F, m, hid, F, R, None, 0,
                                            st))
            check(lib.btl_rope_append_attention(self.q.data_ptr(), self.k.data_ptr(), self.v.data_ptr(), m,
                                                c.n_heads, ctypes.byref(self.caches[li].c), pos, dp,
                                                self.rope_cos.data_ptr(), self.rope_sin.data_ptr(),
                                                self.attn.data_ptr(), self._ws, self._ws_n, st))
            check(lib.btl_linear_group_mode(L["o"], self._y_o, 1, self.attn.data_ptr(), F, m, qd, F, R, None, 0, st))
            check(lib.btl_add_rmsnorm(cur.data_ptr(), self.o.data_ptr(), nxt.data_ptr(), L["n2"], c.eps, m, hid,
                                      self.xn.data_ptr(), st))
            cur, nxt = nxt, cur
            check(lib.btl_linear_group_mode(L["gu"], self._y_gu, 2, self.xn.data_ptr(), F, m, hid, F, R, None, 0, st))
            check(lib.btl_swiglu(self.gate.data_ptr(), self.up.data_ptr(), m * c.intermediate, self.hs.data_ptr(), st))
            check(lib.btl_linear_group_mode(L["down"], self._y_down, 1, self.hs.data_ptr(), F, m, c.intermediate, F,
                                            R, None, 0, st))
            delta = self.down
        last = m - 1
        xf = self.xf if self.dense_head else self.xn
        check(lib.btl_add_rmsnorm(cur[last].data_ptr(), self.down[last].data_ptr(), None,
                                  self.w["norm_f"].data_ptr(), c.eps, 1, hid, xf.data_ptr(), st))
        if self.dense_head:
            check(lib.btl_dense_linear(self.w["lm_head"].data_ptr(), self._head_dt, c.vocab, hid, xf.data_ptr(), 1,
                                       self.logits.data_ptr(), st))
        else:
            check(lib.btl_linear_group_mode(self._head, self._y_logits, 1, xf.data_ptr(), F, 1, hid, F, R, None, 0,
                                            st))

    def reset(self):
        """Llama::reset_state / BitLlama::reset_kv_cache (llama.rs:179-186, 460-468)."""
        for cache in self.caches:
            cache.reset()
        self.pos = 0
        self.graph = None

    def forward_one(self, token):
        """BitLlama::forward_one (llama.rs:201-271): one token at the current position;
        returns the logits [vocab] (a view of the model's buffer)."""
        if self.pos >= self.cfg.max_seq:
            raise ValueError("the cache of %d rows is full" % self.cfg.max_seq)
        self.ids[0] = int(token)
        self._run(1, self.pos, None, self.ids)
        self.pos += 1
        return self.logits[0]

    def prefill(self, ids):
        """The prompt in batches of up to max_rows rows; returns the last logits."""
        ids = torch.as_tensor(np.asarray(ids, dtype=np.int32)).to(self.dev)
        n = ids.numel()
        if n == 0 or self.pos + n > self.cfg.max_seq:
            raise ValueError("prompt of %d tokens does not fit the cache (%d rows, %d used)"
                             % (n, self.cfg.max_seq, self.pos))
        for s in range(0, n, self.max_rows):
            m = min(self.max_rows, n - s)
            self.ids[:m] = ids[s:s + m]
            self._run(m, self.pos, None, self.ids)
            self.pos += m
        return self.logits[0]

    def greedy(self):
        """The greedy pick of the current logits on the device (llama.rs:509-515)
        into self.next_id; returns it as an int (synchronises)."""
        check(lib.btl_greedy_next(self.logits.data_ptr(), self.cfg.vocab, self.next_id.data_ptr(), None, None, 0,
                                  self._stream()))
        return int(self.next_id.item())

    # ------------------------------------------------------- device decode loop
    def _step_device(self):
        """One decode step with the position on the device: the token in next_id at
        position *d_pos through the blocks and the head, then the greedy pick
        (next_id, log[*d_pos + 1], ++*d_pos)."""
        self._run(1, 0, self.d_pos, self.next_id)
        check(lib.btl_greedy_next(self.logits.data_ptr(), self.cfg.vocab, self.next_id.data_ptr(),
                                  self.d_pos.data_ptr(), self.log.data_ptr(), self.log.numel(), self._stream()))

    def capture_decode(self):
        """Capture one device-position decode step in a HIP graph.  Every call of the
        step uses the model's own workspace (sized at construction), so later calls
        of any size elsewhere cannot move memory the graph uses."""
        torch.cuda.synchronize(self.dev)
        g = torch.cuda.CUDAGraph()
        s = torch.cuda.Stream(self.dev)
        with torch.cuda.stream(s):
            with torch.cuda.graph(g, stream=s):
                self._step_device()
        torch.cuda.synchronize(self.dev)
        self.graph = g
        return g

    def start_decode(self):
        """Seed the device loop from the host state: *d_pos = pos, log[pos] = next_id."""
        self.d_pos.fill_(self.pos)
        if self.pos < self.log.numel():
            self.log[self.pos:self.pos + 1].copy_(self.next_id)

    def decode_steps(self, n, use_graph=True):
        """n greedy steps on the device, no host synchronisation in between; the
        tokens accumulate in self.log."""
        if self.pos + n > self.cfg.max_seq:
            raise ValueError("%d steps from position %d overflow the cache of %d rows"
                             % (n, self.pos, self.cfg.max_seq))
        for _ in range(n):
            if use_graph and self.graph is not None:
                self.graph.replay()
            else:
                self._step_device()
        self.pos += n

    def generate(self, prompt_ids, max_tokens, use_graph=True):
        """Llama::stream_completion at temperature 0 (llama.rs:471-530): prefill, then
        greedy decode.  Returns the max_tokens generated ids."""
        self.reset()
        self.prefill(prompt_ids)
        self.greedy()
        start = self.pos
        self.start_decode()
        if max_tokens > 1:
            if use_graph:
                self.capture_decode()
            self.decode_steps(max_tokens - 1, use_graph=use_graph)
        torch.cuda.synchronize(self.dev)
        return self.log[start:start + max_tokens].cpu().numpy().copy()


def random_weights(cfg, device="cuda", seed=0, std=0.02, embed_dtype=torch.float32):
    """Seeded synthetic weights of the architecture: N(0, std) dense weights
    absmean-ternarised on the GPU (btl_pack_device), N(0, 1) embedding rows and
    norm weights 1 + N(0, 0.1) (no checkpoint loading here)."""
    dev = torch.device(device)
    gen = torch.Generator(device=dev)
    gen.manual_seed(seed)
    c = cfg

    def lin(n, k):
        w = torch.randn((n, k), generator=gen, device=dev, dtype=torch.float32) * std
        p = PackedTensor.pack_device(w)
        del w
        return p

    def norm(n):
        return (1.0 + 0.1 * torch.randn((n,), generator=gen, device=dev, dtype=torch.float32)).contiguous()

    kvd = c.n_kv_heads * c.head_dim
    layers = []
    for _ in range(c.n_layers):
        layers.append({"norm1": norm(c.hidden), "norm2": norm(c.hidden),
                       "q": lin(c.n_heads * c.head_dim, c.hidden), "k": lin(kvd, c.hidden), "v": lin(kvd, c.hidden),
                       "o": lin(c.hidden, c.n_heads * c.head_dim), "gate": lin(c.intermediate, c.hidden),
                       "up": lin(c.intermediate, c.hidden), "down": lin(c.hidden, c.intermediate)})
    embed = torch.randn((c.vocab, c.hidden), generator=gen, device=dev, dtype=torch.float32).to(embed_dtype)
    return {"embed": embed.contiguous(), "norm_f": norm(c.hidden), "lm_head": lin(c.vocab, c.hidden),
            "layers": layers}
