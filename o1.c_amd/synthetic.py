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
