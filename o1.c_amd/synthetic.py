"""Random-init weight store of the HiDream-O1 denoiser architecture on the
GPU (the reference loads GGUF packs; no checkpoint exists offline). Names
follow the reference's tensor manifest (forward.c:72-82, block.c:76-88).
Projection weights ~N(0, std) in bf16; RMSNorm gains 1 + N(0, std)."""
import ctypes

import torch

from . import o1hip as H

VOCAB = 151936
TMS_ID = 151673    # <|tms_token|> (generate.c)
PATCH_FEATS = 3072
XE_MID = 1024


def _randn(shape, gen, dev, std, offset=0.0):
    t = torch.empty(shape, dtype=torch.float32, device=dev)
    t.normal_(0.0, std, generator=gen)
    if offset:
        t += offset
    return t.to(torch.bfloat16)


def build_model(n_layers=36, hidden=4096, heads=32, kv_heads=8, ff=12288, head_dim=128,
                vocab=VOCAB, seed=0, std=0.02, device="cuda:0"):
    dev = torch.device(device)
    gen = torch.Generator(device=dev)
    gen.manual_seed(seed)
    t = {}
    L = "model.language_model."
    t[L + "embed_tokens.weight"] = _randn((vocab, hidden), gen, dev, std)
    t["model.t_embedder1.mlp.0.weight"] = _randn((hidden, 256), gen, dev, std)
    t["model.t_embedder1.mlp.0.bias"] = _randn((hidden,), gen, dev, std)
    t["model.t_embedder1.mlp.2.weight"] = _randn((hidden, hidden), gen, dev, std)
    t["model.t_embedder1.mlp.2.bias"] = _randn((hidden,), gen, dev, std)
    t["model.x_embedder.proj1.weight"] = _randn((XE_MID, PATCH_FEATS), gen, dev, std)
    t["model.x_embedder.proj2.weight"] = _randn((hidden, XE_MID), gen, dev, std)
    t["model.x_embedder.proj2.bias"] = _randn((hidden,), gen, dev, std)
    t["model.final_layer2.linear.weight"] = _randn((PATCH_FEATS, hidden), gen, dev, std)
    t["model.final_layer2.linear.bias"] = _randn((PATCH_FEATS,), gen, dev, std)
    t[L + "norm.weight"] = _randn((hidden,), gen, dev, std, 1.0)
    for i in range(n_layers):
        p = f"{L}layers.{i}."
        t[p + "self_attn.q_proj.weight"] = _randn((heads * head_dim, hidden), gen, dev, std)
        t[p + "self_attn.k_proj.weight"] = _randn((kv_heads * head_dim, hidden), gen, dev, std)
        t[p + "self_attn.v_proj.weight"] = _randn((kv_heads * head_dim, hidden), gen, dev, std)
        t[p + "self_attn.o_proj.weight"] = _randn((hidden, heads * head_dim), gen, dev, std)
        t[p + "input_layernorm.weight"] = _randn((hidden,), gen, dev, std, 1.0)
        t[p + "post_attention_layernorm.weight"] = _randn((hidden,), gen, dev, std, 1.0)
        t[p + "mlp.gate_proj.weight"] = _randn((ff, hidden), gen, dev, std)
        t[p + "mlp.up_proj.weight"] = _randn((ff, hidden), gen, dev, std)
        t[p + "mlp.down_proj.weight"] = _randn((hidden, ff), gen, dev, std)
        t[p + "self_attn.q_norm.weight"] = _randn((head_dim,), gen, dev, std, 1.0)
        t[p + "self_attn.k_norm.weight"] = _randn((head_dim,), gen, dev, std, 1.0)
    return t


class Model:
    """Weight store + resolved hd_forward_binding over build_model()."""

    def __init__(self, tensors, n_layers):
        self.tensors = tensors
        self.store = H.WeightStore(tensors)
        self.binding = H.hd_forward_binding()
        st = H.load().hd_forward_resolve(ctypes.byref(self.store.store), n_layers,
                                         ctypes.byref(self.binding))
        H.check_status(st, "hd_forward_resolve")

    def __del__(self):
        try:
            if H._lib is not None and getattr(self, "binding", None) is not None:
                H._lib.hd_forward_binding_free(ctypes.byref(self.binding))
        except (AttributeError, TypeError):     # interpreter shutdown
            pass


# ---- Qwen3-VL vision tower (reference images) ------------------------------
V_HID, V_INTER, V_OUT, V_PATCH = 1152, 4304, 4096, 1536


def build_vision(seed=1, std=0.02, device="cuda:0"):
    """Random-init vision tower under the checkpoint names hd_vision_resolve
    looks up (vision.c:43-130): LayerNorm gains 1 + N(0, 0.1), biases and
    projections N(0, std), position table N(0, 0.5)."""
    dev = torch.device(device)
    gen = torch.Generator(device=dev)
    gen.manual_seed(seed)
    V = "model.visual."
    t = {V + "patch_embed.proj.weight": _randn((V_HID, V_PATCH), gen, dev, std),
         V + "patch_embed.proj.bias": _randn((V_HID,), gen, dev, std),
         V + "pos_embed.weight": _randn((2304, V_HID), gen, dev, 0.5)}
    for i in range(27):
        p = f"{V}blocks.{i}."
        for nm in ("norm1", "norm2"):
            t[p + nm + ".weight"] = _randn((V_HID,), gen, dev, 0.1, 1.0)
            t[p + nm + ".bias"] = _randn((V_HID,), gen, dev, std)
        for nm, (o, k) in (("attn.qkv", (3 * V_HID, V_HID)), ("attn.proj", (V_HID, V_HID)),
                           ("mlp.linear_fc1", (V_INTER, V_HID)), ("mlp.linear_fc2", (V_HID, V_INTER))):
            t[p + nm + ".weight"] = _randn((o, k), gen, dev, std)
            t[p + nm + ".bias"] = _randn((o,), gen, dev, std)
    for pre, nw in [(V + "merger.", V_HID)] + [(f"{V}deepstack_merger_list.{j}.", 4 * V_HID)
                                               for j in range(3)]:
        t[pre + "norm.weight"] = _randn((nw,), gen, dev, 0.1, 1.0)
        t[pre + "norm.bias"] = _randn((nw,), gen, dev, std)
        t[pre + "linear_fc1.weight"] = _randn((4 * V_HID, 4 * V_HID), gen, dev, std)
        t[pre + "linear_fc1.bias"] = _randn((4 * V_HID,), gen, dev, std)
        t[pre + "linear_fc2.weight"] = _randn((V_OUT, 4 * V_HID), gen, dev, std)
        t[pre + "linear_fc2.bias"] = _randn((V_OUT,), gen, dev, std)
    return t


def vision_flops(n):
    """Algorithmic FLOP of one vision forward over n patches (GEMMs at the
    model's widths, attention at head_dim 72)."""
    m = n // 4
    blk = 2 * n * V_HID * (3 * V_HID + V_HID + 2 * V_INTER) + 4 * n * n * V_HID
    merger = 2 * m * (4 * V_HID) * (4 * V_HID + V_OUT)
    return 2 * n * V_PATCH * V_HID + 27 * blk + 4 * merger


class VisionTower:
    """Weight store + hd_vision_resolve binding + workspace for `images`
    reference images of grid_h x grid_w patches; __call__(pixels
    [images*n, 1536]) fills embeds [images*n/4, 4096] and the three deepstack
    outputs (one hd_vision_forward_multi call; hd_vision_forward when
    images == 1)."""

    def __init__(self, tensors, grid_h, grid_w, images=1):
        lib = H.load()
        self.tensors = tensors
        self.store = H.WeightStore(tensors)
        self.binding = H.hd_vision_binding()
        H.check_status(lib.hd_vision_resolve(ctypes.byref(self.store.store), ctypes.byref(self.binding)),
                       "hd_vision_resolve")
        self.gh, self.gw, self.n, self.images = grid_h, grid_w, grid_h * grid_w, images
        dev = next(iter(tensors.values())).device
        self.buf = torch.empty(lib.hd_vision_workspace_bytes_multi(images, self.n), dtype=torch.uint8,
                               device=dev)
        self.tab = torch.empty(lib.hd_vision_tables_bytes(self.n), dtype=torch.uint8, device=dev)
        self.ws = H.hd_vision_workspace()
        self.ws.patch_out = self.buf.data_ptr()
        self.ws.tables = self.tab.data_ptr()
        self.ws.tables_n = -1
        H.check_status(lib.hd_vision_prepare_tables(ctypes.byref(self.ws), self.n, grid_h, grid_w),
                       "hd_vision_prepare_tables")

    def __call__(self, pixels, embeds, deepstack):
        dsp = (ctypes.c_void_p * 3)(*[d.data_ptr() for d in deepstack]) if deepstack else None
        lib = H.load()
        if self.images == 1:
            st = lib.hd_vision_forward(ctypes.byref(self.binding), ctypes.byref(self.ws),
                                       pixels.data_ptr(), self.n, self.gh, self.gw,
                                       embeds.data_ptr(), dsp)
        else:
            st = lib.hd_vision_forward_multi(ctypes.byref(self.binding), ctypes.byref(self.ws),
                                             pixels.data_ptr(), self.images, self.n, self.gh,
                                             self.gw, embeds.data_ptr(), dsp)
        H.check_status(st, "hd_vision_forward")
