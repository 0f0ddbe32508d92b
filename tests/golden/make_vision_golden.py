"""Writes tests/golden/vision_tiny.npz: a tiny random-weight Qwen3-VL vision
tower run in fp32 by transformers (the installed third-party package, not the
reference), as the independent pin of the oracle's vision restatement.

The reference's src/model/vision.c:1-21 states that it reproduces
transformers' Qwen3VLVisionModel stage by stage; this fixture holds that
model's outputs for a 4x6-patch image at a configuration small enough to
commit (depth 3, hidden 32, 2 heads of 16, deepstack after blocks 0 and 2).

Run from the repo root: python tests/golden/make_vision_golden.py
"""
import os

import numpy as np
import torch
from transformers.models.qwen3_vl.configuration_qwen3_vl import Qwen3VLVisionConfig
from transformers.models.qwen3_vl.modeling_qwen3_vl import Qwen3VLVisionModel

OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "vision_tiny.npz")


def main():
    torch.manual_seed(7)
    cfg = Qwen3VLVisionConfig(depth=3, hidden_size=32, hidden_act="gelu_pytorch_tanh",
                              intermediate_size=40, num_heads=2, in_channels=3, patch_size=2,
                              spatial_merge_size=2, temporal_patch_size=2, out_hidden_size=24,
                              num_position_embeddings=16, deepstack_visual_indexes=[0, 2])
    cfg._attn_implementation = "eager"
    model = Qwen3VLVisionModel(cfg).float().eval()
    with torch.no_grad():
        for p in model.parameters():          # O(1) weights so every stage matters
            p.copy_(torch.randn_like(p) * (0.3 if p.ndim > 1 else 0.1))
    gh, gw = 4, 6
    pixels = torch.randn(gh * gw, 3 * 2 * 2 * 2)
    with torch.no_grad():
        out = model(pixels, grid_thw=torch.tensor([[1, gh, gw]]))
    arrays = {"pixels": pixels.numpy(), "grid": np.array([gh, gw]),
              "embeds": out.pooler_output.numpy(),
              "deepstack0": out.deepstack_features[0].numpy(),
              "deepstack1": out.deepstack_features[1].numpy()}
    for name, p in model.state_dict().items():
        arrays["w." + name] = p.detach().numpy().reshape(p.shape[0], -1) if name.endswith(
            "patch_embed.proj.weight") else p.detach().numpy()
    np.savez_compressed(OUT, **arrays)
    print("wrote", OUT, {k: v.shape for k, v in arrays.items() if not k.startswith("w.")})


if __name__ == "__main__":
    main()
