"""Writes the small golden fixtures under tests/golden/.

Sources (nothing here imports or runs reference code):
  * gemm_smoke.json  - the two known-answer cases of the reference's
    tests/unit/test_gemm_smoke.c:104-130 (integer inputs; expected values by
    exact integer arithmetic, then bf16 round-to-nearest-even).
  * positions_s23.json - the position-id known answer quoted in
    src/runtime/sequence.c:97-100 (S=23, T=19, 2x2 grid, fix point 4096).
  * scheduler_sigmas.json - the SIGMAS rows of the reference's scheduler
    oracle dump (tests/unit/oracle_dump.txt: recipe name, steps, shift,
    scheduler kind, sigmas), produced upstream by the Python pipeline.
  * bf16_rne.json - bf16 RNE bit patterns of seeded float32 values produced
    by torch (the library whose conversion the reference emulates,
    support.cu:21-28), including ties and subnormals.
Run: python tests/golden/make_golden.py
"""
import json
import os

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))


def bf16_bits_int(v):
    """RNE of an exactly representable float32 integer value -> bf16 bits."""
    return int(torch.tensor([float(v)], dtype=torch.float32).to(torch.bfloat16).view(torch.int16)[0]) & 0xFFFF


def gemm_smoke():
    cases = []
    X, W = [1, 2, 3, 4], [5, 6, 7, 8]
    cases.append({"name": "2x2", "M": 2, "N": 2, "K": 2, "X": X, "W": W,
                  "Y": [17, 23, 39, 53]})
    M, N, K = 4, 3, 5
    X = list(range(1, M * K + 1))
    W = list(range(1, N * K + 1))
    Y = []
    for m in range(M):
        for n in range(N):
            acc = sum(X[m * K + k] * W[n * K + k] for k in range(K))
            Y.append(acc)
    cases.append({"name": "4x3x5", "M": M, "N": N, "K": K, "X": X, "W": W, "Y_exact": Y,
                  "Y_bf16_bits": [bf16_bits_int(y) for y in Y]})
    return {"source": "tests/unit/test_gemm_smoke.c:104-130", "cases": cases}


def positions():
    T, gh, gw, fp = 19, 2, 2, 4096
    d0 = list(range(T)) + [4096, 4096, 4096, 4096]
    d1 = list(range(T)) + [4096, 4096, 4097, 4097]
    d2 = list(range(T)) + [4096, 4097, 4096, 4097]
    return {"source": "src/runtime/sequence.c:97-100", "S": 23, "text_len": T, "grid_h": gh,
            "grid_w": gw, "fix_point": fp, "pos": [d0, d1, d2]}


def bf16_rne():
    g = torch.Generator().manual_seed(123)
    x = torch.randn(200, generator=g) * torch.exp(torch.randn(200, generator=g) * 8)
    special = torch.tensor([0.0, -0.0, 1.0, 1.00390625, 1.01171875, 1.0078125, 3.0e38, 1e-40,
                            -2.5, 65504.0], dtype=torch.float32)
    # ties: mantissa low half exactly 0x8000 with even / odd upper lsb
    ties = torch.tensor([0x3F808000, 0x3F818000, 0xBF808000, 0x40490000 | 0x8000],
                        dtype=torch.int64).to(torch.int32).view(torch.float32)
    x = torch.cat([x, special, ties])
    bits_in = x.view(torch.int32).tolist()
    out = (x.to(torch.bfloat16).view(torch.int16).to(torch.int32) & 0xFFFF).tolist()
    return {"source": "torch %s float32 -> bfloat16 (RNE)" % torch.__version__,
            "f32_bits": [b & 0xFFFFFFFF for b in bits_in], "bf16_bits": out}


def scheduler_sigmas(path="/root/reference/tests/unit/oracle_dump.txt"):
    recipes = []
    cur = None
    for line in open(path):
        parts = line.split()
        if not parts:
            continue
        if parts[0] == "RECIPE":
            cur = {"name": parts[1], "steps": int(parts[2]), "shift": float(parts[3]),
                   "kind": parts[4], "explicit_timesteps": parts[5] == "True"}
            recipes.append(cur)
        elif parts[0] == "SIGMAS" and cur is not None:
            cur["sigmas"] = [float(v) for v in parts[1:]]
    return {"source": "tests/unit/oracle_dump.txt (RECIPE/SIGMAS rows)", "recipes": recipes}


def scheduler_matrix(path="/root/reference/tests/unit/oracle_dump_matrix.txt"):
    """Per-recipe sigmas, noise scales and one sampler result from the
    upstream scheduler dump (the draws are torch MT19937 seed 1234: z, mo,
    unused, and for flash one more noise, 64 values each, recipe by recipe;
    mo is scaled by 0.3; flash/flow_match record one step, default (UniPC)
    three steps with constant mo)."""
    recipes = []
    cur = None
    for line in open(path):
        parts = line.split()
        if not parts or parts[0].startswith("#"):
            continue
        if parts[0] == "RECIPE":
            cur = {"name": parts[1], "steps": int(parts[2]), "shift": float(parts[3]),
                   "kind": parts[4], "explicit_timesteps": parts[5] == "True"}
            recipes.append(cur)
        elif parts[0] in ("SIGMAS", "NOISESCALE", "STEP") and cur is not None:
            cur[parts[0].lower()] = [float(v) for v in parts[1:]]
    return {"source": "tests/unit/oracle_dump_matrix.txt", "seed": 1234, "n": 64,
            "recipes": recipes}


if __name__ == "__main__":
    for name, fn in (("gemm_smoke.json", gemm_smoke), ("positions_s23.json", positions),
                     ("bf16_rne.json", bf16_rne), ("scheduler_sigmas.json", scheduler_sigmas),
                     ("scheduler_matrix.json", scheduler_matrix)):
        with open(os.path.join(HERE, name), "w") as f:
            json.dump(fn(), f, indent=1)
        print("wrote", name)
