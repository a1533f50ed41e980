"""Device counters of the launches that merge partial results inside the launch,
once their slots run out.  The batched decode's split-K merge counters, the
one-token attention's chunk-merge counters and the greedy pick's state are keyed by
the workspace (or, for the greedy pick, the output word): a key keeps its slot and a
slot never passes to another key, so calls that do not share a workspace never
share counters.  More keys than slots must fall back to routes without counters
(a reduce launch, a second merge launch, one workgroup) and stay bit-exact, also for
the keys that still own slots.  Collected late on purpose: it fills every slot of
the process."""
import ctypes

import numpy as np
import pytest
import torch

import bitlinear as bl
from datagen import activations, weights
from oracle import oracle as orc
from test_gpu_model import Cache, _fill_cache, assert_same, rope_dev, stream

pytestmark = [pytest.mark.gpu,
              pytest.mark.skipif(not torch.cuda.is_available(), reason="needs a GPU")]

DEV = "cuda"


def test_split_merge_counters_beyond_the_slots(tune):
    # 128 slots: 140 workspaces, each used twice, the first ones again at the end
    print("split counters beyond the slots", flush=True)
    tune("BTL_SPLIT_MERGE", 1)
    m, k, n = 4, 14336, 384
    wb, sw = orc.pack(weights(n, k, seed=301))
    pt = bl.PackedTensor(torch.from_numpy(wb).to(DEV), sw, (n, k), DEV)
    x = torch.from_numpy(activations(m, k, seed=302)).to(DEV).to(torch.bfloat16)
    ref = orc.forward_i8(x.float().cpu().numpy(), wb, n, sw)[0]
    wss = [bl.Workspace(m, n, k, device=DEV) for _ in range(140)]
    outs = []
    for ws in wss + wss[:8] + wss[-8:]:
        outs.append(bl.BitLinearHip.forward(x, pt, out_dtype=torch.float32, workspace=ws))
    torch.cuda.synchronize()
    for y in outs:
        assert_same(y, ref, "split-K merge")


def test_attention_merge_counters_beyond_the_slots():
    # 64 slots: 72 workspaces for the one-token attention with the merge in the launch
    print("attention counters beyond the slots", flush=True)
    nh, nkv, hd, S, pos = 8, 2, 128, 256, 130
    rng = np.random.default_rng(303)
    q = rng.standard_normal((1, nh * hd)).astype(np.float32)
    k = (rng.standard_normal((1, nkv * hd)) * 2).astype(np.float32)
    v = rng.standard_normal((1, nkv * hd)).astype(np.float32)
    cos, sin, dc, ds = rope_dev(500000.0, hd, S)
    cache = Cache(nkv, S, hd)
    _fill_cache(cache, S, seed=304)
    qt, kt, vt = (torch.from_numpy(a).to(DEV) for a in (q, k, v))
    ws_bytes = bl.lib.btl_attention_workspace_bytes(1, nh, ctypes.byref(cache.c))
    wss = [torch.empty((ws_bytes + 256,), dtype=torch.uint8, device=DEV) for _ in range(72)]
    outs = []
    for ws in wss + wss[:4]:
        out = torch.full((1, nh * hd), 3.0, device=DEV)
        bl.check(bl.lib.btl_rope_append_attention(qt.data_ptr(), kt.data_ptr(), vt.data_ptr(), 1, nh,
                                                  ctypes.byref(cache.c), pos, None, dc.data_ptr(), ds.data_ptr(),
                                                  out.data_ptr(), ws.data_ptr(), ws_bytes, stream()))
        outs.append(out)
    torch.cuda.synchronize()
    kq, ks, vq, vs = cache.host()
    qr = orc.rope_apply(q[0].reshape(nh, hd), cos[pos], sin[pos]).reshape(-1)
    exp = orc.attn_decode(qr, kq, ks, vq, vs, nh, pos + 1)
    for out in outs:
        assert_same(out[0], exp, "attention")


def test_greedy_state_beyond_the_slots():
    # 64 slots: 72 output words, each with its own pick over a vocabulary-sized row
    print("greedy states beyond the slots", flush=True)
    rng = np.random.default_rng(305)
    x = rng.standard_normal(128256).astype(np.float32)
    x[[1000, 120000]] = 7.5  # a tie: the later index wins
    xt = torch.from_numpy(x).to(DEV)
    nids = [torch.full((1,), -5, dtype=torch.int32, device=DEV) for _ in range(72)]
    for nid in nids + nids[:4]:
        bl.check(bl.lib.btl_greedy_next(xt.data_ptr(), x.size, nid.data_ptr(), None, None, 0, stream()))
    torch.cuda.synchronize()
    for nid in nids:
        assert int(nid.item()) == orc.argmax(x) == 120000
