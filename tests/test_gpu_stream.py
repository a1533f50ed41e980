"""GPU parity of the decode stream (btl_stream_*): every stage output of the
one-launch projection chain, bit for bit, against the oracle run stage by stage
(W1.58-A8 per projection on the bf16-rounded input, bf16 outputs, silu(gate) * up
in f32 then bf16), at small shapes, at the down-projection row-pair geometry, and
at full Llama-3-8B width; repeated launches (the device epoch), a zero input, and
the fault word."""
import numpy as np
import pytest
import torch

import bitlinear as bl
from bitlinear.stream import DecodeStream
from datagen import activations, weights
from oracle import oracle as orc

pytestmark = [pytest.mark.gpu, pytest.mark.skipif(not torch.cuda.is_available(), reason="needs a GPU")]

DEV = "cuda"
NAMES = ("q", "k", "v", "o", "gate", "up", "down")


def bf16r(v):
    return orc.bf16_to_f32(orc.f32_to_bf16(np.asarray(v, np.float32)))


def make_layers(nl, H, I, nkv, seed):
    shapes = {"q": (H, H), "k": (nkv, H), "v": (nkv, H), "o": (H, H), "gate": (I, H), "up": (I, H),
              "down": (H, I)}
    host, dev = [], []
    for l in range(nl):
        hl, dl = {}, {}
        for i, nm in enumerate(NAMES):
            n, k = shapes[nm]
            wb, sw = orc.pack(weights(n, k, seed + 17 * l + i))
            hl[nm] = (wb, n, sw)
            dl[nm] = bl.PackedTensor(torch.from_numpy(wb).to(DEV), sw, (n, k), DEV)
        host.append(hl)
        dev.append(dl)
    return host, dev


def oracle_chain(x, host, H):
    """The stage outputs (f32 values of the bf16 results) of every layer."""
    out = []
    for L in host:
        ys = [orc.forward_i8(x[None], L[nm][0], L[nm][1], L[nm][2])[0][0] for nm in ("q", "k", "v")]
        qkv = bf16r(np.concatenate(ys))
        o = bf16r(orc.forward_i8(qkv[None, :H], *L["o"])[0][0])
        g = orc.forward_i8(o[None], *L["gate"])[0][0]
        u = orc.forward_i8(o[None], *L["up"])[0][0]
        h = bf16r(orc.swiglu(g, u))
        d = bf16r(orc.forward_i8(h[None], *L["down"])[0][0])
        out.append(np.concatenate([qkv, o, h, d]))
        x = d
    return np.concatenate(out)


def run_and_check(ds, host, H, x):
    xt = torch.from_numpy(orc.f32_to_bf16(x).view(np.int16)).to(DEV).view(torch.bfloat16)
    st = torch.full((ds.words,), 0x7FC0, dtype=torch.int16, device=DEV).view(torch.bfloat16)
    y = ds.run(xt, stage_out=st)
    torch.cuda.synchronize()
    bl.check_faults()
    ref = orc.f32_to_bf16(oracle_chain(x, host, H))
    got = st.view(torch.int16).cpu().numpy().view(np.uint16)
    bad = np.flatnonzero(got != ref)
    assert bad.size == 0, "%d stage words differ, first at %d: %#x vs %#x" % (bad.size, bad[0], got[bad[0]], ref[bad[0]])
    assert np.array_equal(y.view(torch.int16).cpu().numpy().view(np.uint16), ref[-H:])
    return y


# (layers, hidden, intermediate, k/v rows): down rows in groups of 4 (I <= 4096) or of
# 2 (I > 4096); q|k|v groups crossing the k and v boundaries; most workgroups idle
SHAPES = [(3, 256, 512, 64), (2, 256, 4352, 128), (2, 512, 1024, 128), (1, 1024, 2048, 256)]


@pytest.mark.parametrize("nl,H,I,nkv", SHAPES)
def test_stream_matches_oracle(nl, H, I, nkv):
    print("stream", nl, H, I, nkv, flush=True)
    host, dev = make_layers(nl, H, I, nkv, seed=H + I)
    ds = DecodeStream(dev)
    try:
        for rep in range(2):  # a second launch must not see the first's words (epoch)
            run_and_check(ds, host, H, bf16r(activations(1, H, seed=rep + 3)[0]))
        run_and_check(ds, host, H, np.zeros(H, np.float32))
    finally:
        ds.close()


def test_stream_llama3_8b_width():
    # full Llama-3-8B projection shapes, two layers
    print("stream llama3-8b width", flush=True)
    H, I, nkv = 4096, 14336, 1024
    host, dev = make_layers(2, H, I, nkv, seed=5)
    ds = DecodeStream(dev)
    try:
        for rep in range(2):
            run_and_check(ds, host, H, bf16r(activations(1, H, seed=40 + rep)[0]))
    finally:
        ds.close()


def test_stream_wait_budget_is_reported(tune):
    # a zero time budget: every cross-workgroup wait gives up at once, the launch
    # still finishes and btl_check_faults reports it; the default budget is exact again
    print("stream fault word", flush=True)
    host, dev = make_layers(1, 256, 512, 64, seed=9)
    ds = DecodeStream(dev)
    try:
        xt = torch.from_numpy(orc.f32_to_bf16(bf16r(activations(1, 256, seed=1)[0])).view(np.int16)).to(DEV)
        tune("BTL_WAIT_SPIN", 0)
        ds.run(xt.view(torch.bfloat16))
        with pytest.raises(bl.BitLinearError) as ei:
            bl.check_faults()
        assert ei.value.status == bl.BTL_ERR_FAULT and "stream" in str(ei.value)
        tune("BTL_WAIT_SPIN", 1 << 22)
        run_and_check(ds, host, 256, bf16r(activations(1, 256, seed=2)[0]))
    finally:
        ds.close()
