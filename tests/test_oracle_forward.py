"""Pins the oracle's whole-denoiser forward (o1o_forward / o1o_forward_visual,
the restatement of forward.c:253-397) against an independent torch fp64
statement written from the reference file, not from the oracle:

- t-embedder: t*1000 -> 256-d sinusoid, cos half then sin half with
  freq_p = exp(-ln(1e4) p / 128) (gemm.cu:530-545) -> te0 + bias -> SiLU
  (act.cu:13-19) -> te2 + bias (forward.c:253-266);
- token gather, ids outside [0, vocab) read row 0 (embed.cu:24-26);
- masked scatter of the image embeddings into the text rows, then the
  timestep-token substitution on top of it (forward.c:272-291,
  vision_kernels.cu:344-363, embed.cu:60-70);
- x_embedder proj1 (no bias) -> proj2 + bias (forward.c:301-313);
- blocks (the layer statement of test_oracle.torch_block), DeepStack add on
  the image-pad rows after layers 0, 1, 2 (forward.c:363-370,
  vision_kernels.cu:377-401);
- final RMSNorm -> head + bias (forward.c:388-397).

Each of four plausible misreadings (SiLU dropped, DeepStack one layer late,
the timestep token applied before the scatter, proj2 bias dropped) moves the
result by more than 1e-2, so a shared misreading cannot pass."""
import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import oracle as orc
from tests.common import make_forward_weights, make_block_weights, grid_pos, rel_l2, bf16, TMS
from tests.test_oracle import torch_block

NL, HID, H, KV, FF, D = 4, 256, 2, 1, 512, 128
VOC = 1000
THETA = 1e4


def torch_forward(fw, ids, vin, t, pos, tms_id, visual=None, ar_len=0,
                  drop_silu=False, ds_shift=0, tms_first=False, drop_xe2_bias=False):
    """forward.c:253-397 in torch fp64 (the sinusoid in fp32 as the
    reference's kernel computes it: its argument reaches 1000 rad)."""
    dd = lambda a: torch.as_tensor(np.asarray(a)).double()
    T, I = len(ids), vin.shape[0]
    S = T + I
    # t-embedder
    half = 128
    p = torch.arange(half, dtype=torch.float32)
    freq = torch.exp(-math.log(10000.0) * p / half)
    arg = torch.tensor(t * 1000.0, dtype=torch.float32) * freq
    sinus = torch.cat([torch.cos(arg), torch.sin(arg)]).double()
    th = sinus @ dd(fw["te0_w"]).T + dd(fw["te0_b"])
    temb = th if drop_silu else F.silu(th)
    temb = temb @ dd(fw["te2_w"]).T + dd(fw["te2_b"])
    # text rows
    tab = dd(fw["embed_tokens"])
    idt = torch.as_tensor(ids)
    safe = torch.where((idt < 0) | (idt >= tab.shape[0]), torch.zeros_like(idt), idt)
    h_text = tab[safe].clone()
    is_tms = idt == tms_id
    if tms_first:
        h_text[is_tms] = temb
    if visual is not None:
        emb, ds, vm = visual
        vmt = torch.as_tensor(vm[:T]).bool()
        h_text[vmt] = dd(emb)[: int(vmt.sum())]
    if not tms_first:
        h_text[is_tms] = temb
    # image rows
    b2 = 0.0 if drop_xe2_bias else dd(fw["xe2_b"])
    h_img = (dd(vin) @ dd(fw["xe1_w"]).T) @ dd(fw["xe2_w"]).T + b2
    h = torch.cat([h_text, h_img]).float()
    for l, bw in enumerate(fw["blocks"]):
        h = torch.from_numpy(torch_block(h, pos, bw, H, KV, D, THETA, ar_len=ar_len))
        if visual is not None:
            li = l - ds_shift
            if 0 <= li < 3 and ds[li] is not None:
                vms = torch.as_tensor(vm).bool()
                h = h.double()
                h[vms] += dd(ds[li])
                h = h.float()
    hn = F.rms_norm(h.double(), (HID,), dd(fw["fnorm_w"]), 1e-6)
    return (hn @ dd(fw["fl_w"]).T + dd(fw["fl_b"])).numpy()


def weights():
    fw = make_forward_weights(NL, HID, H, KV, FF, D, seed=21, vocab=VOC)
    g = torch.Generator().manual_seed(22)
    # biases and the t-embedder at a scale where dropping any one of them
    # is visible at the output (the checkpoint's are O(1) too)
    for k, std in (("te0_b", 1.0), ("te2_b", 0.5), ("xe2_b", 0.5), ("fl_b", 0.5)):
        fw[k] = bf16(torch.randn(fw[k].shape, generator=g) * std)
    fw["te0_w"] = bf16(torch.randn(fw["te0_w"].shape, generator=g) * 0.2)
    fw["te2_w"] = bf16(torch.randn(fw["te2_w"].shape, generator=g) * 0.1)
    # blocks far from the identity, so the layer an add lands after matters
    fw["blocks"] = [make_block_weights(HID, H, KV, FF, D, seed=40 + i, std=0.06) for i in range(NL)]
    return fw


def inputs(T=20, gh=6, gw=7, seed=3):
    rng = np.random.default_rng(seed)
    ids = rng.integers(0, VOC, T).astype(np.int64)
    ids[2] = -5            # below the table: row 0
    ids[5] = VOC + 17      # past the table: row 0
    ids[T - 1] = TMS       # outside this table's range; substitution wins
    vin = bf16(torch.from_numpy(rng.standard_normal((gh * gw, 3072)).astype(np.float32))).numpy()
    return ids, vin, grid_pos(T, gh, gw)


def np_fw(fw):
    out = {k: v.numpy() for k, v in fw.items() if k != "blocks"}
    out["blocks"] = [{k: v.numpy() for k, v in b.items()} for b in fw["blocks"]]
    return out


def cfg(ar_len=0):
    return orc.block_cfg(H, KV, HID, FF, D, theta=THETA, faithful=0, ar_len=ar_len)


@pytest.mark.parametrize("ar_len", [0, 19])
def test_forward_oracle_vs_torch(ar_len):
    fw = weights()
    ids, vin, pos = inputs()
    if ar_len:
        pos[:, :len(ids)] = np.arange(len(ids))[None]
    t = 0.5
    want = torch_forward(fw, ids, vin, t, pos, TMS, ar_len=ar_len)
    got = orc.forward(np_fw(fw), cfg(ar_len), ids, vin, t, pos, TMS)
    assert rel_l2(got, want) < 1e-5, rel_l2(got, want)
    # the timestep token inside the table's range: substitution, not a lookup
    ids2 = ids.copy()
    ids2[7] = 11
    want2 = torch_forward(fw, ids2, vin, t, pos, 11, ar_len=ar_len)
    got2 = orc.forward(np_fw(fw), cfg(ar_len), ids2, vin, t, pos, 11)
    assert rel_l2(got2, want2) < 1e-5


def visual_case(fw, ids, T, S, seed=9):
    """Image-pad rows 1..17 of the text (one of them also the timestep
    token), image embeddings for them and three DeepStack tensors."""
    g = torch.Generator().manual_seed(seed)
    vm = np.zeros(S, np.uint8)
    vm[1:18] = 1
    ids = ids.copy()
    ids[10] = TMS          # image-pad row that is also the timestep token
    nv = int(vm.sum())
    emb = bf16(torch.randn(nv, HID, generator=g)).numpy()
    ds = [bf16(torch.randn(nv, HID, generator=g) * 2.0).numpy() for _ in range(3)]
    return ids, (emb, ds, vm)


def test_forward_visual_oracle_vs_torch():
    fw = weights()
    ids, vin, pos = inputs()
    T, S = len(ids), len(ids) + vin.shape[0]
    ids, vis = visual_case(fw, ids, T, S)
    want = torch_forward(fw, ids, vin, 0.3, pos, TMS, visual=vis)
    got = orc.forward(np_fw(fw), cfg(), ids, vin, 0.3, pos, TMS, visual=vis)
    assert rel_l2(got, want) < 1e-5, rel_l2(got, want)


def test_forward_pin_rejects_misreadings():
    """Each misreading moves the whole-forward output by > 1e-2 from the
    oracle's, so the 1e-5 agreement above pins all four."""
    fw = weights()
    ids, vin, pos = inputs()
    T, S = len(ids), len(ids) + vin.shape[0]
    idv, vis = visual_case(fw, ids, T, S)
    got = orc.forward(np_fw(fw), cfg(), idv, vin, 0.3, pos, TMS, visual=vis)
    for kw in (dict(drop_silu=True), dict(ds_shift=1), dict(tms_first=True),
               dict(drop_xe2_bias=True)):
        bad = torch_forward(fw, idv, vin, 0.3, pos, TMS, visual=vis, **kw)
        assert rel_l2(got, bad) > 1e-2, (kw, rel_l2(got, bad))
