"""Benchmark of the DIMQ packed-index hot path on one MI355X.

Default run: the two halves of the BASELINE metric on one JSON line.
* Headline (``value``): BASELINE configs[1] (cfg2), the ResNet-18 layer1 3x3
  conv with a 2-bit per-output-channel codebook: x fp16 [32,64,56,56] (ReLU of
  N(0,1)), W [64,64,3,3] Kaiming-normal, stride 1, pad 1, no bias, y fp32.  One
  step = one LUT conv launch over one batch.
* ``models.vit_b16``: BASELINE configs[3], the ViT-B/16 bs64 forward with its
  48 Linears 4-bit, in images/s with the MFMA roofline over the forward's
  FLOPs and the dequantized fp32 model timed on the host beside it.
Single workloads: ``--config cfg1|cfg2|cfg5|codec|vit|resnet18|w4a4_linear|w4a4_conv|w4a4_linear_q|w4a4_conv_q``.

Timing: inputs are resident in HBM before the timed region; R buffer sets
(> 512 MB in total, so the 256 MB MALL cannot serve repeats) are rotated; the
steps are captured once in a HIP graph (torch.cuda.CUDAGraph) so the GPU runs
them back to back, and HIP events on the launch stream bracket the K timed
steps.  Prints ONE JSON line.
"""

from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time
from pathlib import Path

import torch

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0
MFMA_F16_PEAK_TFLOPS = 2500.0
METRIC = "LUT-GEMM/conv TFLOP/s + % roofline; ViT-B/16 4-bit bs64 images/s"


# ---------------------------------------------------------------------------
# workloads
# ---------------------------------------------------------------------------

def _conv_weight_cfg2(g):
    w = torch.randn(64, 64, 3, 3, generator=g) * math.sqrt(2.0 / 576.0)  # kaiming_normal_, fan_in 576
    return w


def make_cfg2(dev, rotations, layout="nchw", variant="auto"):
    from dimq_amd import ops
    from dimq_amd.codebook import assign_indices, init_centers_per_channel
    from dimq_amd.export import pack_indices

    g = torch.Generator().manual_seed(1)
    w = _conv_weight_cfg2(g)
    centers = init_centers_per_channel(w, 4)                      # [64, 4] fp32
    idx = assign_indices(w, centers)                              # GPU kernel
    packed = pack_indices(idx, 2).to(dev)                         # GPU kernel
    prepared = ops.prepare_conv_weight(packed, 2, (64, 64, 3, 3))  # one-time kernel-layout repack
    cb = centers.to(dev)
    mf = torch.channels_last if layout == "nhwc" else torch.contiguous_format
    xs = [torch.relu(torch.randn(32, 64, 56, 56, generator=g)).half().to(dev).contiguous(memory_format=mf)
          for _ in range(rotations)]

    def step(i):
        return ops.dimq_conv2d_codebook(xs[i], packed, cb, 2, None, (64, 64, 3, 3), (1, 1), (1, 1), (1, 1), 1,
                                        out_dtype=torch.float32, prepared_weight=prepared, variant=variant)

    x_bytes = 32 * 64 * 56 * 56 * 2
    y_bytes = 32 * 64 * 56 * 56 * 4
    alg_bytes = x_bytes + y_bytes + packed.numel() + cb.numel() * 4
    flops = 2.0 * 32 * 56 * 56 * 64 * 64 * 9

    def cpu_step(sample_batch):
        import oracle
        return oracle.conv2d_dequant_reference(xs[0][:sample_batch].cpu().float(), packed.cpu(), 2, centers,
                                               (64, 64, 3, 3), None, 1, 1, 1, 1)

    def check():
        import oracle
        y = step(0)
        ref = oracle.conv2d_dequant_reference(xs[0].cpu().float(), packed.cpu(), 2, centers, (64, 64, 3, 3), None,
                                              1, 1, 1, 1)
        return oracle.rel_err(y, ref)

    return dict(
        name="cfg2",
        workload="ResNet-18 layer1 conv3x3: x fp16 [32,64,56,56] (ReLU N(0,1)), W [64,64,3,3] Kaiming-normal, "
                 "2-bit per-output-channel codebook (4 centroids/row, quantile init), stride 1, pad 1, no bias, "
                 f"y fp32 {layout.upper()}",
        step=step, flops=flops, alg_bytes=alg_bytes, bound="hbm", dtype="fp16",
        unit="TFLOP/s", per_step_units=flops / 1e12, cpu_step=cpu_step, cpu_full_batch=32, check=check,
        extra_config={"global_batch": 32, "in_shape": [32, 64, 56, 56], "weight_shape": [64, 64, 3, 3],
                      "bits": 2, "codebook": "per_channel", "layout": layout},
        per_set_bytes=x_bytes + y_bytes,
    )


def make_cfg1(dev, rotations, variant="auto"):
    from dimq_amd import ops
    from dimq_amd.codebook import assign_indices, init_centers_per_channel
    from dimq_amd.export import pack_indices

    g = torch.Generator().manual_seed(0)
    w = torch.randn(3072, 768, generator=g) * 0.02
    b = torch.randn(3072, generator=g) * 0.02
    centers = init_centers_per_channel(w, 16)
    packed = pack_indices(assign_indices(w, centers), 4).to(dev)
    cb = centers.to(dev)
    bias = b.to(dev)
    xs = [torch.randn(1576, 768, generator=g).to(dev) for _ in range(rotations)]

    def step(i):
        return ops.dimq_linear_codebook(xs[i], packed, cb, 4, bias, 3072, 768, out_dtype=torch.float32,
                                        variant=variant)

    alg_bytes = 1576 * 768 * 4 + packed.numel() + cb.numel() * 4 + 3072 * 4 + 1576 * 3072 * 4
    flops = 2.0 * 1576 * 3072 * 768

    def cpu_step(sample_rows):
        import oracle
        return oracle.linear_dequant_reference(xs[0][:sample_rows].cpu(), packed.cpu(), 4, centers, 3072, 768, b)

    def check():
        import oracle
        return oracle.rel_err(step(0), oracle.linear_dequant_reference(xs[0].cpu(), packed.cpu(), 4, centers, 3072,
                                                                       768, b))

    return dict(
        name="cfg1",
        workload="ViT-B/16 MLP fc1 Linear: X fp32 [1576,768], W [3072,768] N(0,0.02), 4-bit per-output-channel "
                 "codebook (16 centroids/row, quantile init), bias, Y fp32",
        step=step, flops=flops, alg_bytes=alg_bytes, bound="hbm", dtype="fp16",
        unit="TFLOP/s", per_step_units=flops / 1e12, cpu_step=cpu_step, cpu_full_batch=1576, check=check,
        extra_config={"M": 1576, "N": 3072, "K": 768, "bits": 4, "codebook": "per_channel"},
        per_set_bytes=1576 * 768 * 4 + 1576 * 3072 * 4,
    )


_QUANT_CACHE = {}


def make_cfg5(dev, rotations, M=16, variant="auto"):
    from dimq_amd import ops
    from dimq_amd.codebook import assign_indices, init_centers_per_channel
    from dimq_amd.export import pack_indices

    g = torch.Generator().manual_seed(4)
    w = torch.randn(4096, 4096, generator=g) * 0.02
    if "cfg5" not in _QUANT_CACHE:  # the same seeded weights for every M: quantize once per process
        c = init_centers_per_channel(w, 8)
        _QUANT_CACHE["cfg5"] = (c, pack_indices(assign_indices(w, c), 3).cpu())
    centers, packed_cpu = _QUANT_CACHE["cfg5"]
    cb = centers.to(dev)
    # weights rotate too (6.3 MB packed each) so that repeats stream from HBM
    packs = [packed_cpu.to(dev)]
    for _ in range(rotations - 1):
        packs.append(packs[0].clone())
    xs = [torch.randn(M, 4096, generator=g).bfloat16().to(dev) for _ in range(rotations)]

    def step(i):
        return ops.dimq_linear_codebook(xs[i], packs[i], cb, 3, None, 4096, 4096, out_dtype=torch.float32,
                                        variant=variant)

    alg_bytes = packs[0].numel() + cb.numel() * 4 + M * 4096 * 2 + M * 4096 * 4
    flops = 2.0 * M * 4096 * 4096

    def cpu_step(sample_rows):
        import oracle
        return oracle.linear_dequant_reference(xs[0][:sample_rows].cpu().float(), packs[0].cpu(), 3, centers, 4096,
                                               4096)

    def check():
        import oracle
        return oracle.rel_err(step(0), oracle.linear_dequant_reference(xs[0].cpu().float(), packs[0].cpu(), 3,
                                                                       centers, 4096, 4096))

    return dict(
        name=f"cfg5_m{M}",
        workload=f"decode GEMV: X bf16 [{M},4096], W [4096,4096] N(0,0.02), 3-bit per-output-channel codebook "
                 "(8 centroids/row), Y fp32",
        step=step, flops=flops, alg_bytes=alg_bytes, bound="hbm", dtype="fp16",
        unit="TFLOP/s", per_step_units=flops / 1e12, cpu_step=cpu_step, cpu_full_batch=M, check=check,
        extra_config={"M": M, "N": 4096, "K": 4096, "bits": 3, "codebook": "per_channel"},
        per_set_bytes=packs[0].numel() + M * 4096 * 6,
    )


def make_codec(dev, rotations, direction="unpack"):
    from dimq_amd import ops

    n = 1 << 27
    g = torch.Generator().manual_seed(5)
    idx = torch.randint(0, 8, (n,), generator=g, dtype=torch.uint8)
    base = idx.to(dev)
    packed0 = ops.pack_bits(base, 3)
    srcs = [base if i == 0 else base.clone() for i in range(rotations)] if direction == "pack" else \
        [packed0 if i == 0 else packed0.clone() for i in range(rotations)]

    if direction == "pack":
        def step(i):
            return ops.pack_bits(srcs[i], 3)
    else:
        def step(i):
            return ops.unpack_bits(srcs[i], n, 3)

    alg_bytes = n + n * 3 // 8

    idx_np = idx.numpy()
    packed_np = packed0.cpu().numpy()

    def cpu_step(sample):
        import oracle
        if direction == "pack":
            return oracle.pack_bits(idx_np[:sample], 3)
        sample -= sample % 8                      # whole 3-byte groups
        return oracle.unpack_bits(packed_np[:sample * 3 // 8], sample, 3)

    def check():
        back = ops.unpack_bits(ops.pack_bits(base, 3), n, 3)
        return 0.0 if torch.equal(back, base) else 1.0

    return dict(
        name=f"codec_{direction}",
        workload=f"3-bit codec {direction}: 2^27 uniform random indices <-> 50,331,648 packed bytes",
        step=step, flops=0.0, alg_bytes=alg_bytes, bound="hbm", dtype="u8",
        unit="GB/s", per_step_units=alg_bytes / 1e9, cpu_step=cpu_step, cpu_full_batch=n, check=check,
        extra_config={"numel": n, "bits": 3},
        per_set_bytes=alg_bytes, cpu_cores=1,
        cpu_desc="the oracle's C LSB-first bit packer/unpacker (one thread; the reference's CPU codec is "
                 "torch slicing, dimq_backend/export.py:38-78)",
    )


def _cast_float_params(model, dtype):
    """Unquantized parameters (embeddings, LayerNorm, head, ...) to `dtype`; codebook layers keep fp32 codebooks."""
    from dimq_amd.modules import DIMQCodebookConv2d, DIMQCodebookLinear
    for mod in model.modules():
        if isinstance(mod, (DIMQCodebookConv2d, DIMQCodebookLinear)):
            continue
        for name, prm in list(mod._parameters.items()):
            if prm is not None:
                mod._parameters[name] = torch.nn.Parameter(prm.detach().to(dtype), requires_grad=False)
    return model


def _model_workload(name, workload, dev, rotations, qmodel, xs_cpu, flops_per_image, dtype_name, mf, extra,
                    check_images=2):
    """Shared plumbing of the end-to-end model workloads: graph-replayed forward, images/s.  The parity check
    runs the first ``check_images`` images on both sides; enough for the timed kernel paths to be the checked
    ones (the ViT's Linears take the pre-decoded path from 2048 rows on)."""
    batch = xs_cpu.shape[0]
    xdt = torch.bfloat16 if dtype_name == "bf16" else torch.float16
    xs = [xs_cpu.to(dev).to(xdt).contiguous(memory_format=mf) for _ in range(rotations)]
    qmodel.eval()

    @torch.no_grad()
    def step(i):
        return qmodel(xs[i])

    def cpu_model():
        import oracle
        if "cpu" not in _model_workload.cache:
            _model_workload.cache["cpu"] = oracle.dequantized_model(qmodel)
        return _model_workload.cache["cpu"]

    @torch.no_grad()
    def cpu_step(sample):
        return cpu_model()(xs_cpu[:sample].float())

    @torch.no_grad()
    def check():
        import oracle
        n = check_images
        ref = cpu_model()(xs_cpu[:n].float())
        out = qmodel(xs[0][:n]).float().cpu()
        return oracle.rel_err(out, ref)

    return dict(
        name=name, workload=workload, step=step, flops=flops_per_image * batch, alg_bytes=0, bound="mfma",
        dtype=dtype_name, unit="images/s", per_step_units=float(batch), cpu_step=cpu_step, cpu_full_batch=batch,
        check=check, extra_config={"global_batch": batch, **extra},
        per_set_bytes=xs_cpu.numel() * 2,
    )


_model_workload.cache = {}


def make_vit(dev, rotations):
    from dimq_amd.bench_models import quantize_vit, vit_b16, vit_flops
    g = torch.Generator().manual_seed(3)
    xs_cpu = torch.randn(64, 3, 224, 224, generator=g)
    m = vit_b16().to(dev)
    m = _cast_float_params(quantize_vit(m, 4, out_dtype=torch.bfloat16), torch.bfloat16)
    return _model_workload(
        "vit_b16", "ViT-B/16 forward, bs64, 3x224x224 N(0,1): qkv/proj/fc1/fc2 4-bit per-output-channel codebooks "
        "(N(0,0.02) weights); patch embedding, LayerNorm, residual stream and head in bf16, the tensors that only "
        "feed a codebook GEMM and the qkv -> attention (SDPA) -> proj link in fp16",
        dev, rotations, m, xs_cpu, vit_flops(1), "bf16", torch.contiguous_format,
        {"model": "vit_b16", "image": 224, "bits": 4, "codebook": "per_channel", "parity_images": 11},
        check_images=11)  # 11 x 197 = 2167 rows: the pre-decoded path and batched decode the timed forward takes


def make_resnet18(dev, rotations):
    from dimq_amd.bench_models import quantize_resnet18, resnet18, resnet18_flops
    g = torch.Generator().manual_seed(2)
    xs_cpu = torch.randn(128, 3, 224, 224, generator=g)
    m = resnet18().to(dev).to(memory_format=torch.channels_last)
    m = _cast_float_params(quantize_resnet18(m, out_dtype=torch.float16), torch.float16)
    return _model_workload(
        "resnet18", "ResNet-18 forward, bs128, 3x224x224 N(0,1), BN folded: 8-bit stem and fc, 2-bit 3x3 convs, "
        "4-bit 1x1 downsample (per-output-channel codebooks); fp16 channels_last activations",
        dev, rotations, m, xs_cpu, resnet18_flops(1), "fp16", torch.channels_last,
        {"model": "resnet18", "image": 224, "bits": "8/2/4/8", "codebook": "per_channel"})


def make_copy(dev, rotations):
    """Calibration only: a plain 256 MiB device-to-device copy, whose HBM bytes are known exactly.

    Used to scale the FETCH_SIZE / WRITE_SIZE counters of the other workloads."""
    n = 256 << 20
    srcs = [torch.randint(0, 255, (n,), dtype=torch.uint8, device=dev) for _ in range(rotations)]
    dst = torch.empty(n, dtype=torch.uint8, device=dev)

    def step(i):
        return dst.copy_(srcs[i])

    def check():
        return 0.0 if torch.equal(step(0), srcs[0]) else 1.0

    def cpu_step(sample):
        return srcs[0][:sample].cpu().clone()

    return dict(
        name="copy", workload="calibration: 256 MiB uint8 device copy (torch copy_)",
        step=step, flops=0.0, alg_bytes=2 * n, bound="hbm", dtype="u8",
        unit="GB/s", per_step_units=2 * n / 1e9, cpu_step=cpu_step, cpu_full_batch=n, check=check,
        extra_config={"bytes": n}, per_set_bytes=n,
    )


def make_w4a4(dev, rotations, op="linear", chained=False):
    """The reference's own W4A4 ops (dimq::linear_lut / dimq::conv2d_lut) at the cfg1 / cfg2 shapes.

    One 16-entry per-layer fp16 codebook (the packed exporter's format,
    dimq_backend/export.py:167,217), u4 activations with scale/zero point;
    y fp32.  One step = one op call (activation quantization pass + GEMM/conv).
    chained: the layer inside a chain of W4A4 layers -- its input arrives as the
    fp16 codes a - zp from the layer before, and it writes the next layer's
    codes (ReLU, then u4 quantization fused into its epilogue); the conv's
    kernel-layout weight is prepared once, as a loaded layer holds it.
    """
    from dimq_amd import ops
    from dimq_amd.codebook import assign_indices
    from dimq_amd.export import pack_indices

    g = torch.Generator().manual_seed(6)
    cb16 = torch.linspace(-0.06, 0.06, 16).half()
    cb_dev = cb16.to(dev)
    scale, zp = 0.25, 8
    if op == "linear":
        N, K, M = 3072, 768, 1576
        w = torch.randn(N, K, generator=g) * 0.02
        b = torch.randn(N, generator=g) * 0.02
        packed = pack_indices(assign_indices(w, cb16.float()), 4).to(dev)
        bias = b.to(dev)
        xs = [torch.randn(M, K, generator=g).to(dev) for _ in range(rotations)]

        def step(i):
            return ops.dimq_linear_lut(xs[i], packed, cb_dev, scale, zp, bias, N, K)

        x_bytes, y_bytes = M * K * 4, M * N * 4
        if chained:
            xqs = [ops.quantize_activation_f16(x, scale, zp) for x in xs]

            def step(i):
                return ops.dimq_linear_lut_q(xqs[i], packed, cb_dev, scale, bias, N, K, activation="relu",
                                             out_act=(0.125, 3))

            x_bytes, y_bytes = M * K * 2, M * N * 2
        flops = 2.0 * M * N * K
        full = M

        def cpu_step(rows):
            import oracle
            return oracle.linear_a4_dequant_reference(xs[0][:rows].cpu(), packed.cpu(), cb16.float(), scale, zp, N, K,
                                                      b)

        def check():
            import oracle
            ref = oracle.linear_lut(xs[0].cpu(), packed.cpu(), cb16.float(), scale, zp, b, N, K)
            if chained:  # the same kernels with a float output
                return oracle.rel_err(ops.dimq_linear_lut_q(xqs[0], packed, cb_dev, scale, bias, N, K),
                                      torch.from_numpy(ref))
            return oracle.rel_err(step(0), torch.from_numpy(ref))

        workload = ("reference W4A4 linear_lut at the cfg1 shape: X fp32 [1576,768], W [3072,768] 4-bit, one 16-entry "
                    "fp16 codebook, u4 activations (scale 0.25, zp 8), bias, Y fp32")
        extra = {"M": M, "N": N, "K": K, "bits": 4, "codebook": "per_layer_fp16", "op": "linear_lut"}
    else:
        shape = (64, 64, 3, 3)
        w = _conv_weight_cfg2(g)
        packed = pack_indices(assign_indices(w.reshape(64, -1), cb16.float()), 4).to(dev)
        xs = [torch.relu(torch.randn(32, 64, 56, 56, generator=g)).half().to(dev) for _ in range(rotations)]

        def step(i):
            return ops.dimq_conv2d_lut(xs[i], packed, cb_dev, scale, zp, None, shape, (1, 1), (1, 1), (1, 1), 1)

        x_bytes, y_bytes = 32 * 64 * 56 * 56 * 2, 32 * 64 * 56 * 56 * 4
        if chained:
            xqs = [ops.quantize_activation_f16(x, scale, zp) for x in xs]
            prep = ops.prepare_conv_weight(packed, 4, shape)

            def step(i):
                return ops.dimq_conv2d_lut_q(xqs[i], packed, cb_dev, scale, None, shape, 1, 1,
                                             prepared_weight=prep, activation="relu", out_act=(0.125, 3))

            y_bytes = 32 * 64 * 56 * 56 * 2
        flops = 2.0 * 32 * 56 * 56 * 64 * 64 * 9
        full = 32

        def cpu_step(batch):
            import oracle
            return oracle.conv2d_a4_dequant_reference(xs[0][:batch].cpu().float(), packed.cpu(), cb16.float(), scale,
                                                      zp, shape, None, 1, 1, 1, 1)

        def check():
            import oracle
            ref = oracle.conv2d_lut(xs[0].cpu().float(), packed.cpu(), cb16.float(), scale, zp, None, shape, 1, 1, 1,
                                    1)
            if chained:  # the same kernels with a float output
                return oracle.rel_err(ops.dimq_conv2d_lut_q(xqs[0], packed, cb_dev, scale, None, shape, 1, 1,
                                                            prepared_weight=prep), torch.from_numpy(ref))
            return oracle.rel_err(step(0), torch.from_numpy(ref))

        workload = ("reference W4A4 conv2d_lut at the cfg2 shape: x fp16 [32,64,56,56] (ReLU N(0,1)), W [64,64,3,3] "
                    "4-bit, one 16-entry fp16 codebook, u4 activations (scale 0.25, zp 8), stride 1, pad 1, y fp32 NCHW")
        extra = {"global_batch": 32, "in_shape": [32, 64, 56, 56], "weight_shape": list(shape), "bits": 4,
                 "codebook": "per_layer_fp16", "op": "conv2d_lut"}
    if chained:
        workload = (workload.replace("reference W4A4 ", "chained W4A4 ") +
                    "; input as fp16 codes a - zp from the previous layer, output the next layer's fp16 codes "
                    "(ReLU, scale 0.125, zp 3) from the fused epilogue")
        extra = dict(extra, op=extra["op"] + "_q", chained=True)
    alg_bytes = x_bytes + y_bytes + packed.numel() + 32
    return dict(
        name=f"w4a4_{op}" + ("_q" if chained else ""), workload=workload, step=step, flops=flops, alg_bytes=alg_bytes, bound="hbm",
        dtype="fp16", unit="TFLOP/s", per_step_units=flops / 1e12, cpu_step=cpu_step, cpu_full_batch=full,
        check=check, extra_config=extra, per_set_bytes=x_bytes + y_bytes,
        cpu_desc="the reference's CPU path: u4 activations and W_hat = C[idx] dequantized, then torch CPU fp32 "
                 "F.linear / F.conv2d (reference.py:91-144)",
    )


VIT_LINEARS = {  # name: N, K, activation dtype, epilogue, output dtype (as in the bs64 forward)
    "qkv": (2304, 768, torch.float16, None, torch.float16),
    "proj": (768, 768, torch.float16, "residual", torch.bfloat16),
    "fc1": (3072, 768, torch.float16, "gelu", torch.float16),
    "fc2": (768, 3072, torch.float16, "residual", torch.bfloat16),
}


def make_vit_linear(dev, rotations, shape="qkv", path="auto"):
    """One Linear of the ViT-B/16 bs64 forward at M = 64 x 197 tokens, 4-bit per-channel codebook of N(0, 0.02)
    weights, with its fused epilogue; path "fused" calls the C entry without a workspace (the shared-decode
    tile) instead of the pre-decoded path the ops take."""
    from dimq_amd import _C, ops
    from dimq_amd.codebook import assign_indices, init_centers_per_channel
    from dimq_amd.export import pack_indices

    N, K, xdt, epi, odt = VIT_LINEARS[shape]
    M = 64 * 197
    g = torch.Generator().manual_seed(N + K)
    w = torch.randn(N, K, generator=g) * 0.02
    b = torch.randn(N, generator=g) * 0.02
    centers = init_centers_per_channel(w, 16)
    packed = pack_indices(assign_indices(w, centers), 4).to(dev)
    cb, bias = centers.to(dev), b.to(dev)
    xs = [torch.randn(M, K, generator=g).to(xdt).to(dev) for _ in range(rotations)]
    res = (torch.randn(M, N, generator=g) * 0.5).bfloat16().to(dev) if epi == "residual" else None
    ys = [torch.empty(M, N, dtype=odt, device=dev) for _ in range(rotations)]
    dt = {torch.float32: 0, torch.float16: 1, torch.bfloat16: 2}

    def step(i):
        if path == "auto":
            return ops.dimq_linear_codebook(xs[i], packed, cb, 4, bias, N, K, out_dtype=odt, residual=res,
                                            activation="gelu" if epi == "gelu" else None)
        rc = _C.lib.dimq_linear_codebook_ex(xs[i].data_ptr(), dt[xdt], M, K, packed.data_ptr(), packed.numel(), 4,
                                            cb.data_ptr(), 0, N, 16, bias.data_ptr(), 0, N, ys[i].data_ptr(), dt[odt],
                                            0 if res is None else res.data_ptr(), 2, 2 if epi == "gelu" else 0, 0,
                                            torch.cuda.current_stream().cuda_stream)
        if rc != 0:
            raise RuntimeError(_C.lib.dimq_last_error())
        return ys[i]

    flops = 2.0 * M * N * K

    def ref(rows):
        import oracle
        r = oracle.linear_dequant_reference(xs[0][:rows].float().cpu(), packed.cpu(), 4, centers, N, K, b)
        if epi == "residual":
            r = r + res[:rows].float().cpu()
        elif epi == "gelu":
            r = torch.nn.functional.gelu(r)
        return r

    def check():
        import oracle
        return oracle.rel_err(step(0).float().cpu()[:2048], ref(2048))

    return dict(
        name=f"vit_{shape}",
        workload=f"ViT-B/16 bs64 {shape} Linear: X {str(xdt)[6:]} [{M},{K}], W [{N},{K}] N(0,0.02) 4-bit per-channel "
                 f"codebook, bias{', ' + epi if epi else ''}, Y {str(odt)[6:]} ({path} path)",
        step=step, flops=flops, alg_bytes=M * K * xdt.itemsize + packed.numel() + M * N * odt.itemsize,
        bound="mfma", dtype="fp16", unit="TFLOP/s", per_step_units=flops / 1e12,
        cpu_step=lambda rows: ref(rows), cpu_full_batch=M, check=check,
        extra_config={"M": M, "N": N, "K": K, "bits": 4, "codebook": "per_channel", "path": path},
        per_set_bytes=M * K * xdt.itemsize + M * N * odt.itemsize,
    )


FIXED_ROTATIONS = {"vit": 4, "resnet18": 4}
WORKLOADS = {"cfg2": make_cfg2, "cfg1": make_cfg1, "cfg5": make_cfg5, "codec": make_codec, "copy": make_copy,
             "vit": make_vit, "resnet18": make_resnet18,
             "w4a4_linear": lambda dev, r: make_w4a4(dev, r, "linear"),
             "w4a4_conv": lambda dev, r: make_w4a4(dev, r, "conv"),
             "w4a4_linear_q": lambda dev, r: make_w4a4(dev, r, "linear", chained=True),
             "w4a4_conv_q": lambda dev, r: make_w4a4(dev, r, "conv", chained=True),
             "vit_linear": make_vit_linear}


# ---------------------------------------------------------------------------
# timing
# ---------------------------------------------------------------------------

def time_gpu(wl, rotations, steps, warmup):
    """Captures `rotations` steps in one HIP graph, replays it; returns ms per step from HIP events."""
    step = wl["step"]
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for i in range(rotations):      # eager warm-up outside capture
            step(i)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()

    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for i in range(rotations):
            step(i)
    # exactly `steps` timed steps: whole replays of the rotation graph, then a graph of the first `rem` sets
    # (the sets the warm-up touched longest ago when steps < rotations)
    replays, rem = divmod(steps, rotations)
    graph_rem = None
    if rem:
        graph_rem = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph_rem):
            for i in range(rem):
                step(i)
    for _ in range(max(1, warmup // rotations)):
        graph.replay()
    torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(replays):
        graph.replay()
    if graph_rem is not None:
        graph_rem.replay()
    end.record()
    torch.cuda.synchronize()
    ms = start.elapsed_time(end) / steps
    return ms, steps


def time_cpu(wl, budget_s=15.0):
    """Times the oracle's CPU path (dequantize, then torch CPU fp32 conv/linear) on a bounded sample."""
    threads = len(os.sched_getaffinity(0))
    torch.set_num_threads(threads)
    full = wl["cpu_full_batch"]
    sample = full
    t0 = time.perf_counter()
    wl["cpu_step"](sample)
    one = time.perf_counter() - t0
    # shrink the sample until one call takes at most ~budget/8
    while one > budget_s / 8 and sample > 1:
        sample = max(1, sample // 2)
        t0 = time.perf_counter()
        wl["cpu_step"](sample)
        one = time.perf_counter() - t0
    for _ in range(2):
        wl["cpu_step"](sample)
    times = []
    t_end = time.perf_counter() + budget_s * 0.6
    while len(times) < 10 or (time.perf_counter() < t_end and len(times) < 50):
        t0 = time.perf_counter()
        wl["cpu_step"](sample)
        times.append(time.perf_counter() - t0)
        if len(times) >= 10 and time.perf_counter() > t_end:
            break
    times.sort()
    med = times[len(times) // 2]
    frac = sample / full
    value = wl["per_step_units"] * frac / med
    used = wl.get("cpu_cores", torch.get_num_threads())
    return dict(value=value, unit=wl["unit"], cores=used, kind="port",
                sample=f"{sample}/{full} of one step ({wl['name']}), median of {len(times)} runs after 3 warm-ups; "
                       f"{wl.get('cpu_desc', 'oracle dequantize + torch CPU fp32')}",
                cpu_model=host_cpu_model(), threads_used=used, cpus_available=threads,
                host=host_id())


def host_cpu_model():
    """Full CPU model string of the host that ran the baseline (/proc/cpuinfo)."""
    try:
        info = {}
        n = 0
        for line in open("/proc/cpuinfo"):
            if ":" not in line:
                continue
            k, v = (t.strip() for t in line.split(":", 1))
            n += k == "processor"
            info.setdefault(k, v)
        return (f"{info.get('model name', '?')}, family {info.get('cpu family', '?')} model {info.get('model', '?')} "
                f"stepping {info.get('stepping', '?')}, {info.get('cache size', '?')} cache, "
                f"{info.get('cpu MHz', '?')} MHz ({n} logical CPUs visible)")
    except OSError:
        return "unknown"


def host_id():
    """The machine's hostname and the GPU's name, so baselines of different rounds can be told apart."""
    import socket
    gpu = torch.cuda.get_device_name(0) if torch.cuda.is_available() else "none"
    return f"{socket.gethostname()} / {gpu}"


def run_workload(args, config, dev, steps, warmup, cpu_budget_s=15.0):
    """Builds one workload, checks it against the oracle, times it (HIP graph replays, HIP events) and its
    CPU baseline; returns the fields of its JSON line."""
    make = WORKLOADS[config]
    kw = {}
    if config == "cfg5":
        kw["M"] = args.m
    if config in ("cfg1", "cfg5", "cfg2"):
        kw["variant"] = args.variant
    if config == "codec":
        kw["direction"] = args.direction
    if config == "cfg2":
        kw["layout"] = args.layout
    if config == "vit_linear":
        kw["shape"] = args.shape
        kw["path"] = args.path
    # rotate buffer sets totalling > 512 MB
    if config in FIXED_ROTATIONS:
        # end-to-end models: inputs rotate over a few sets; the packed weights are re-read every step
        rotations = FIXED_ROTATIONS[config]
    else:
        probe = make(dev, 1, **kw)
        rotations = max(2, min(64, math.ceil(512e6 / probe["per_set_bytes"]) + 1))
        del probe
    if args.rotations > 0:
        rotations = args.rotations
    torch.cuda.empty_cache()
    wl = make(dev, rotations, **kw)
    if "variant" in kw:
        wl["extra_config"]["variant"] = kw["variant"]

    err = None if args.no_check else wl["check"]()
    ms, steps = time_gpu(wl, rotations, steps, warmup)
    sec = ms / 1e3
    value = wl["per_step_units"] / sec
    if wl["bound"] == "hbm":
        achieved = wl["alg_bytes"] / sec / 1e9
        roof = {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": None}
    else:
        achieved = wl["flops"] / sec / 1e12
        roof = {"bound": "mfma", "achieved": round(achieved, 2), "peak": MFMA_F16_PEAK_TFLOPS, "unit": "TFLOP/s",
                "frac": round(achieved / MFMA_F16_PEAK_TFLOPS, 4), "traffic": None}
    traffic_file = ROOT / "profiles" / f"traffic_{wl['name']}.json"
    if traffic_file.exists():
        roof["traffic"] = json.loads(traffic_file.read_text()).get("traffic_bytes_per_launch")
    cpu = None if args.no_cpu else time_cpu(wl, cpu_budget_s)
    out = {
        "metric": METRIC,
        "metric_part": "images/s" if wl["unit"] == "images/s" else "LUT-GEMM/conv TFLOP/s + % roofline",
        "value": round(value, 4),
        "unit": wl["unit"],
        "n_gpus": 1,
        "steps": steps,
        "warmup": warmup,
        "ms_per_step": round(ms, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": wl["dtype"],
        "data": "synthetic (seeded CPU torch.Generator, copied to HBM before timing)",
        "config": {"workload": wl["workload"], "name": wl["name"], "rotated_buffer_sets": rotations,
                   "algorithmic_bytes_per_step": wl["alg_bytes"], "flops_per_step": wl["flops"],
                   "parity_max_rel_err": err, **wl["extra_config"]},
        "roofline": roof,
        "cpu_baseline": cpu,
    }
    del wl
    torch.cuda.empty_cache()
    return out


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=1600)
    ap.add_argument("--warmup", type=int, default=160)
    ap.add_argument("--config", default=None, choices=sorted(WORKLOADS),
                    help="one workload (default: cfg2 headline plus the ViT-B/16 bs64 forward on the same line)")
    ap.add_argument("--m", type=int, default=16, help="rows for cfg5")
    ap.add_argument("--direction", default="unpack", choices=["pack", "unpack"])
    ap.add_argument("--layout", default="nchw", choices=["nchw", "nhwc"], help="cfg2 activation layout")
    ap.add_argument("--variant", default="auto", choices=["auto", "small_m", "mfma"],
                    help="cfg1/cfg5: force the LUT-gather (small_m) or dequant+MFMA kernel family; cfg2 (nhwc): "
                         "mfma forces the implicit-GEMM tiles over the LDS-halo kernel")
    ap.add_argument("--shape", default="qkv", choices=sorted(VIT_LINEARS), help="vit_linear: which Linear")
    ap.add_argument("--path", default="auto", choices=["auto", "fused"],
                    help="vit_linear: the ops' path (pre-decoded weights) or the no-workspace shared-decode tile")
    ap.add_argument("--rotations", type=int, default=0,
                    help="buffer sets to rotate (0 = enough for > 512 MB; smaller values let the MALL serve repeats)")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-check", action="store_true")
    args = ap.parse_args()

    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path (every box has one GPU). "
              "Run with --gpus 1.", file=sys.stderr)
        sys.exit(2)

    dev = torch.device("cuda:0")
    if args.config is not None:
        out = run_workload(args, args.config, dev, args.steps, args.warmup)
    else:
        out = run_workload(args, "cfg2", dev, args.steps, args.warmup)
        keep = ("value", "unit", "ms_per_step", "steps", "dtype", "config", "roofline", "cpu_baseline")
        # second half of the metric: the ViT-B/16 bs64 forward (a few graph replays of the whole forward)
        vit = run_workload(args, "vit", dev, max(4, min(args.steps, 40)), max(1, min(args.warmup, 8)),
                           cpu_budget_s=12.0)
        out["models"] = {"vit_b16": {"metric_part": vit["metric_part"], **{k: vit[k] for k in keep}}}
        # every other BASELINE config on the same line, each with its own roofline and CPU baseline
        out["configs"] = {}
        for name, config, kw, steps in DEFAULT_EXTRA:
            sub = argparse.Namespace(**{**vars(args), **kw})
            n = steps(args.steps)
            print(f"[bench] {name}: {n} steps", file=sys.stderr, flush=True)
            r = run_workload(sub, config, dev, n, max(args.warmup, 2), cpu_budget_s=6.0)
            out["configs"][name] = {k: r[k] for k in keep}
    out.pop("metric_part", None)
    print(json.dumps(out), flush=True)


# the default line's "configs" map: name, workload, its options, timed steps as a function of --steps (the
# kernel-sized configs time at least 200 launches so that one event pair brackets >= ~1 ms of GPU work)
DEFAULT_EXTRA = [
    ("cfg1", "cfg1", {}, lambda k: max(k, 200)),
    ("cfg5_m1", "cfg5", {"m": 1}, lambda k: max(k, 200)),
    ("cfg5_m4", "cfg5", {"m": 4}, lambda k: max(k, 200)),
    ("cfg5_m16", "cfg5", {"m": 16}, lambda k: max(k, 200)),
    ("codec_pack", "codec", {"direction": "pack"}, lambda k: max(k, 40)),
    ("codec_unpack", "codec", {"direction": "unpack"}, lambda k: max(k, 40)),
    ("resnet18", "resnet18", {}, lambda k: max(4, min(k, 40))),
]


if __name__ == "__main__":
    main()
