"""Writes the golden vectors under tests/golden/ (run: python tests/golden/make_golden.py).

The reference (fengchao32/DIMQ) stores no vectors: its tests are seeded
recipes and equivalences (dimq_cuda_backend/tests/test_reference_and_export.py,
test_cuda_ops.py).  The vectors here are computed from formulations that are
independent of the C oracle they check:

* codec: a pure-Python bit-list construction of the LSB-first stream (index i
  occupies bits [b*i, b*i+b)), plus the hand-derived u4 vectors that follow the
  nibble rule of dimq_backend/export.py:43;
* nearest-centre assignment, u4 activation quantization, product table and the
  W4A4 / weight-only Linear and Conv2d recipes: torch CPU library routines
  (argmin, round, F.linear, F.conv2d) evaluated the way the reference's
  reference.py / dimq.py do.
"""

from __future__ import annotations

import json
import random
from pathlib import Path

import numpy as np
import torch
import torch.nn.functional as F

OUT = Path(__file__).resolve().parent


def bitlist_pack(indices, bits):
    stream = []
    for v in indices:
        for j in range(bits):
            stream.append((v >> j) & 1)
    while len(stream) % 8:
        stream.append(0)
    out = []
    for i in range(0, len(stream), 8):
        out.append(sum(bit << j for j, bit in enumerate(stream[i:i + 8])))
    return bytes(out)


def codec_vectors():
    cases = []
    hand = [
        (4, [i % 16 for i in range(17)], "10 32 54 76 98 ba dc fe 00"),
        (4, [(i * 7) % 16 for i in range(16)], "70 5e 3c 1a f8 d6 b4 92"),
        (3, [1, 2, 3, 4, 5, 6, 7, 0], "d1 58 1f"),
        (3, list(range(8)), "88 c6 fa"),
        (3, [7] * 8, "ff ff ff"),
        (2, [0, 1, 2, 3], "e4"),
        (2, [3, 2, 1, 0, 1], "1b 01"),
        (8, [0, 255, 17, 128], "00 ff 11 80"),
    ]
    for bits, idx, hexs in hand:
        assert bitlist_pack(idx, bits).hex(" ") == hexs, (bits, idx)
        cases.append({"bits": bits, "indices": idx, "packed": hexs, "source": "hand"})
    rng = random.Random(1234)
    for bits in (2, 3, 4, 8):
        for n in (0, 1, 2, 3, 5, 7, 8, 9, 15, 16, 17, 31, 32, 33, 63, 64, 65, 127, 128, 129, 257, 1000):
            idx = [rng.randrange(1 << bits) for _ in range(n)]
            cases.append({"bits": bits, "indices": idx, "packed": bitlist_pack(idx, bits).hex(" "),
                          "source": "bitlist"})
    # the reference's GPU recipe (test_cuda_ops.py:34): (arange(257)*7) % 16
    idx = [(i * 7) % 16 for i in range(257)]
    cases.append({"bits": 4, "indices": idx, "packed": bitlist_pack(idx, 4).hex(" "), "source": "ref-recipe"})
    return cases


def hardquant_vectors():
    cases = []
    # ties: exact binary midpoints -> the lower index wins (first minimum).
    w = torch.tensor([-2.0, -1.5, -1.0, -0.5, -0.25, 0.0, 0.25, 0.5, 1.0, 1.5, 2.0, 0.75, -0.75])
    c = torch.tensor([-1.0, 0.0, 1.0])
    idx = ((w[:, None] - c[None, :]) ** 2).argmin(1)
    cases.append({"w": w.tolist(), "centers": c.tolist(), "idx": idx.tolist(), "source": "ties"})
    assert idx.tolist() == [0, 0, 0, 0, 1, 1, 1, 1, 2, 2, 2, 2, 0]
    # the reference test recipe (tests/test_dimq_math.py:35-43)
    w = torch.linspace(-2.0, 2.0, 101)
    idx = ((w[:, None] - c[None, :]) ** 2).argmin(1)
    cases.append({"w": w.tolist(), "centers": c.tolist(), "idx": idx.tolist(), "source": "ref-recipe"})
    # duplicated centres: the first copy wins
    w = torch.tensor([0.1, 0.3, 0.5, 0.9])
    c = torch.tensor([0.0, 0.5, 0.5, 1.0])
    idx = ((w[:, None] - c[None, :]) ** 2).argmin(1)
    cases.append({"w": w.tolist(), "centers": c.tolist(), "idx": idx.tolist(), "source": "dup-centres"})
    # random, per K in {4, 8, 16, 256}
    g = torch.Generator().manual_seed(7)
    for K in (4, 8, 16, 256):
        w = torch.randn(300, generator=g) * 0.05
        c = (torch.randn(K, generator=g) * 0.05).sort().values
        idx = ((w[:, None] - c[None, :]) ** 2).argmin(1)
        cases.append({"w": w.tolist(), "centers": c.tolist(), "idx": idx.tolist(), "source": f"random-K{K}"})
    return cases


def actquant_vectors():
    cases = []
    # exact ties: x / s lands on k + 0.5; round-half-to-even.
    x = torch.tensor([0.125, 0.375, 0.625, -0.125, -0.375, -0.625, 1.875, -1.875, 100.0, -100.0, 0.0, -0.0])
    q = torch.clamp(torch.round(x.float() / 0.25) + 8, 0, 15).to(torch.uint8)
    assert q.tolist() == [8, 10, 10, 8, 6, 6, 15, 0, 15, 0, 8, 8]
    cases.append({"x": x.tolist(), "scale": 0.25, "zp": 8, "q": q.tolist(), "source": "ties"})
    g = torch.Generator().manual_seed(11)
    for s, zp in ((0.2, 7), (0.125, 8), (1.0, 8), (0.0731, 3), (1.0 / 3.0, 0)):
        x = torch.randn(512, generator=g) * 1.5
        q = torch.clamp(torch.round(x.float() / float(s)) + int(zp), 0, 15).to(torch.uint8)
        cases.append({"x": x.tolist(), "scale": s, "zp": zp, "q": q.tolist(), "source": "torch-cpu"})
    return cases


def product_table_vectors():
    # recipe of dimq_cuda_backend/tests/test_cuda_ops.py:45-48
    cb = torch.linspace(-1.0, 1.0, 16, dtype=torch.float16)
    a = torch.arange(16, dtype=torch.float32)
    table = cb.float()[:, None] * (0.125 * (a - 8))[None, :]
    assert table[0, 0].item() == 1.0 and table[15, 15].item() == 0.875
    assert table[7, 3].item() == 0.04180908203125
    return [{"codebook": cb.float().tolist(), "codebook_dtype": "float16", "scale": 0.125, "zp": 8,
             "table": table.tolist()}]


def w4a4_recipes():
    """The reference's LUT-vs-dequant recipes with CPU-generated inputs."""
    out = {}
    torch.manual_seed(3)
    x = torch.randn(4, 11)
    cb = torch.linspace(-0.5, 0.5, 16)
    idx = torch.randint(0, 16, (6, 11), dtype=torch.uint8)
    bias = torch.randn(6)
    xq = torch.clamp(torch.round(x / 0.2) + 7, 0, 15)
    y = F.linear(0.2 * (xq - 7), cb[idx.long()], bias)
    out["linear"] = {"x": x.tolist(), "codebook": cb.tolist(), "indices": idx.tolist(), "bias": bias.tolist(),
                     "scale": 0.2, "zp": 7, "y": y.tolist()}
    torch.manual_seed(4)
    x = torch.randn(2, 3, 6, 7)
    cb = torch.linspace(-0.75, 0.75, 16)
    idx = torch.randint(0, 16, (5, 3, 3, 3), dtype=torch.uint8)
    bias = torch.randn(5)
    xq = torch.clamp(torch.round(x / 0.25) + 7, 0, 15)
    y = F.conv2d(0.25 * (xq - 7), cb[idx.long()], bias, (2, 1), (1, 1), (1, 1), 1)
    out["conv2d"] = {"x": x.tolist(), "codebook": cb.tolist(), "indices": idx.tolist(), "bias": bias.tolist(),
                     "scale": 0.25, "zp": 7, "stride": [2, 1], "padding": [1, 1], "dilation": [1, 1], "groups": 1,
                     "y": y.tolist()}
    return out


def weight_only_recipes():
    """Per-channel multi-bit weight-only recipes: Y = X W_hat^T + b (fp32, CPU)."""
    out = {}
    g = torch.Generator().manual_seed(21)
    for bits in (2, 3, 4, 8):
        N, K, M = 5, 13, 3
        Kc = 1 << bits
        cb = torch.randn(N, Kc, generator=g).sort(dim=1).values * 0.1
        idx = torch.randint(0, Kc, (N, K), generator=g, dtype=torch.uint8)
        x = torch.randn(M, K, generator=g)
        bias = torch.randn(N, generator=g)
        y = F.linear(x, torch.gather(cb, 1, idx.long()), bias)
        out[f"linear_b{bits}"] = {"bits": bits, "x": x.tolist(), "codebook": cb.tolist(), "indices": idx.tolist(),
                                  "bias": bias.tolist(), "y": y.tolist()}
    return out


def main():
    (OUT / "codec_vectors.json").write_text(json.dumps(codec_vectors()))
    (OUT / "hardquant_vectors.json").write_text(json.dumps(hardquant_vectors()))
    (OUT / "actquant_vectors.json").write_text(json.dumps(actquant_vectors()))
    (OUT / "product_table_vectors.json").write_text(json.dumps(product_table_vectors()))
    (OUT / "w4a4_recipes.json").write_text(json.dumps(w4a4_recipes()))
    (OUT / "weight_only_recipes.json").write_text(json.dumps(weight_only_recipes()))
    print("wrote", sorted(p.name for p in OUT.glob("*.json")))


if __name__ == "__main__":
    np.random.seed(0)
    main()
