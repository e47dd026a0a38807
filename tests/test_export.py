"""The drop-in checkpoint path: dimq_compact -> dimq_packed_lut export, reload,
module replacement and forward.

CPU tests build compact checkpoints in the layout of
quant/export_dimq.py:56-108 (per-layer 16-centre codebooks for the reference's
W4A4 format, per-channel b-bit codebooks for the weight-only format 2), export
them with the host path and check the reference's own assertions
(dimq_cuda_backend/tests/test_reference_and_export.py:76-83) plus a bit-level
round trip of every layer's indices through oracle.unpack_bits.  GPU tests
replace the layers of a model with the runtime modules the checkpoint
describes and compare the forward with the oracle.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch
import torch.nn as nn

import oracle
from tests.conftest import announce


def _nearest(w, centers):
    """First-minimum argmin of (w - c)^2, torch on the CPU (the reference's expression, quant/dimq.py:214-215)."""
    rows = w.reshape(w.shape[0], -1)
    c = centers if centers.dim() == 2 else centers[None, :].expand(rows.shape[0], -1)
    return ((rows[:, :, None] - c[:, None, :]) ** 2).argmin(dim=2).to(torch.uint8).reshape(w.shape)


def _compact(model, bits_for, per_channel=True, bias_in_state=True):
    """A dimq_compact checkpoint of every Conv2d / Linear of `model` that bits_for(name, module) quantizes."""
    from dimq_amd.codebook import init_centers_1d, init_centers_per_channel
    layers, skip = {}, set()
    for name, mod in model.named_modules():
        if not isinstance(mod, (nn.Conv2d, nn.Linear)):
            continue
        bits = bits_for(name, mod)
        if bits is None:
            continue
        w = mod.weight.detach().float()
        K = 1 << bits
        centers = init_centers_per_channel(w, K) if per_channel else init_centers_1d(w, K)
        layers[name] = {"shape": list(w.shape), "bits": bits, "centers": centers,
                        "indices": _nearest(w, centers), "dequantized_weight_dtype": "float32"}
        skip.add(f"{name}.weight")
    state = {k: v.detach().cpu() for k, v in model.state_dict().items() if k not in skip}
    if not bias_in_state:
        state = {k: v for k, v in state.items() if not k.endswith(".bias")}
    return {"format": "dimq_compact",
            "model_meta": {"num_quantized_layers": len(layers), "quantized_layer_names": list(layers)},
            "quant_cfg": {"w_bits": 4}, "layers": layers, "non_quantized_state_dict": state}


class _Net(nn.Module):
    def __init__(self):
        super().__init__()
        self.conv1 = nn.Conv2d(3, 16, 3, 1, 1)
        self.conv2 = nn.Conv2d(16, 32, 3, 2, 1)
        self.down = nn.Conv2d(16, 32, 1, 2, 0)
        self.fc = nn.Linear(32 * 4 * 4, 10)

    def forward(self, x):
        x = torch.relu(self.conv1(x))
        x = torch.relu(self.conv2(x) + self.down(x))
        return self.fc(torch.flatten(x, 1))


def _net(seed=0):
    torch.manual_seed(seed)
    return _Net()


def test_export_reference_w4a4_layout(tmp_path):
    from dimq_amd.export import export_packed_dimq_checkpoint, infer_module_hparams
    m = _net()
    compact = _compact(m, lambda n, mod: 4, per_channel=False)
    src = tmp_path / "compact.pth"
    torch.save(compact, src)
    out = tmp_path / "packed.pt"
    state = export_packed_dimq_checkpoint(src, out, layer_hparams=infer_module_hparams(m))
    assert out.exists()
    # test_reference_and_export.py:76-83
    assert state["format"] == "dimq_packed_lut"
    assert state["activation_quantization"] == "uniform_affine_u4"
    assert len(state["layers"]) == 4
    first = state["layers"]["conv1"]
    assert first["bit_w"] == 4
    assert first["bit_a"] == 4
    assert first["codebook"].numel() == 16
    assert first["packed_weight"].dtype == torch.uint8
    assert first["packed_weight"].numel() == (first["weight_numel"] + 1) // 2
    # format-1 keys, uncalibrated default qparams (export.py:114-125), conv geometry from the hparams
    assert state["format_version"] == 1 and state["weight_encoding"] == "packed_u4_indices"
    assert first["act_scale"] == 1.0 and first["act_zero_point"] == 8
    conv2 = state["layers"]["conv2"]
    assert conv2["layout"] == "conv_kcrs" and conv2["stride"] == [2, 2] and conv2["padding"] == [1, 1]
    assert state["layers"]["fc"]["layout"] == "linear_nk"
    assert state["layers"]["fc"]["in_features"] == 512 and state["layers"]["fc"]["out_features"] == 10
    # the file holds only tensors and plain containers: it loads without unpickling code
    loaded = torch.load(out, map_location="cpu", weights_only=True)
    for name, layer in compact["layers"].items():
        e = loaded["layers"][name]
        idx = oracle.unpack_bits(e["packed_weight"].numpy(), e["weight_numel"], 4)
        assert np.array_equal(idx, layer["indices"].reshape(-1).numpy()), name
        assert torch.equal(e["codebook"], layer["centers"].reshape(-1).half())
        assert torch.equal(e["bias"], m.state_dict()[f"{name}.bias"].half())


@pytest.mark.parametrize("bits", [2, 3, 4, 8])
def test_export_weight_only_per_channel(tmp_path, bits):
    from dimq_amd.export import export_packed_dimq_checkpoint, infer_module_hparams
    m = _net(bits)
    compact = _compact(m, lambda n, mod: bits, per_channel=True)
    out = tmp_path / f"packed_b{bits}.pt"
    state = export_packed_dimq_checkpoint(compact, out, layer_hparams=infer_module_hparams(m),
                                          codebook_dtype=torch.float32)
    loaded = torch.load(out, map_location="cpu", weights_only=True)
    assert loaded["format_version"] == 2 and loaded["activation_quantization"] == "none"
    assert loaded["weight_encoding"] == "packed_lsb_first_indices"
    for name, layer in compact["layers"].items():
        e = loaded["layers"][name]
        assert e["bit_w"] == bits and e["bit_a"] is None and e["activation_quantization"] == "none"
        assert e["codebook_granularity"] == "per_channel"
        assert tuple(e["codebook"].shape) == (layer["shape"][0], 1 << bits)
        assert e["packed_weight"].numel() == math.ceil(e["weight_numel"] * bits / 8)
        idx = oracle.unpack_bits(e["packed_weight"].numpy(), e["weight_numel"], bits)
        assert np.array_equal(idx, layer["indices"].reshape(-1).numpy()), name
    assert state["layers"]["down"]["padding"] == [0, 0] and state["layers"]["down"]["kernel_size"] == [1, 1]


def test_export_mixed_widths_and_bias_from_state_dict(tmp_path):
    """Per-layer widths picked by the number of centres (8 -> 3 bits, 256 -> 8 bits); biases found in the
    compact checkpoint's non-quantized state dict when no hparams are given; default padding k // 2."""
    from dimq_amd.export import export_packed_dimq_checkpoint
    m = _net(5)
    compact = _compact(m, lambda n, mod: 8 if isinstance(mod, nn.Linear) else 3)
    state = export_packed_dimq_checkpoint(compact, tmp_path / "p.pt", codebook_dtype=torch.float32)
    assert {n: e["bit_w"] for n, e in state["layers"].items()} == {"conv1": 3, "conv2": 3, "down": 3, "fc": 8}
    assert state["layers"]["conv1"]["padding"] == [1, 1] and state["layers"]["conv1"]["stride"] == [1, 1]
    for name in compact["layers"]:
        assert torch.equal(state["layers"][name]["bias"], m.state_dict()[f"{name}.bias"].float())


def test_export_errors(tmp_path):
    from dimq_amd.export import export_packed_dimq_checkpoint
    m = _net(1)
    with pytest.raises(ValueError, match="dimq_compact"):
        export_packed_dimq_checkpoint({"format": "other"}, tmp_path / "x.pt")
    c = _compact(m, lambda n, mod: 2)
    with pytest.raises(ValueError, match="expects 16 learned centers"):
        export_packed_dimq_checkpoint(c, tmp_path / "x.pt", weight_only=False)
    c = _compact(m, lambda n, mod: 4, per_channel=False)
    c["layers"]["fc"]["indices"] = c["layers"]["fc"]["indices"].clone()
    c["layers"]["fc"]["indices"][0, 0] = 16
    with pytest.raises(ValueError, match=r"indices outside \[0, 15\]"):
        export_packed_dimq_checkpoint(c, tmp_path / "x.pt")
    c = _compact(m, lambda n, mod: 4, per_channel=False)
    with pytest.raises(KeyError, match="missing activation qparams"):
        export_packed_dimq_checkpoint(c, tmp_path / "x.pt", act_qparams={"conv1": {"scale": 0.1, "zero_point": 3}})


def test_host_pack_unpack_and_assign_match_oracle():
    """The exporter's host path against the oracle's packer and the reference's argmin expression."""
    from dimq_amd.export import assign_weight_indices, pack_indices, unpack_indices
    g = torch.Generator().manual_seed(4)
    for bits in (2, 3, 4, 8):
        for n in (1, 7, 8, 9, 1001):
            idx = torch.randint(0, 1 << bits, (n,), generator=g, dtype=torch.uint8)
            packed = pack_indices(idx, bits)
            assert bytes(packed.numpy()) == bytes(oracle.pack_bits(idx, bits)), (bits, n)
            assert torch.equal(unpack_indices(packed, n, bits), idx)
    w = torch.randn(33, 19, generator=g)
    cb = torch.arange(16, dtype=torch.float32) * 0.25 - 2.0   # dyadic centres: exact midpoints
    w[0, 0] = -1.125                                            # midway between cb[3] and cb[4]: the lower wins
    got = assign_weight_indices(w, cb)
    assert torch.equal(got, ((w.reshape(-1, 1) - cb[None, :]) ** 2).argmin(1).to(torch.uint8).reshape(w.shape))
    assert int(got[0, 0]) == 3


# ---------------------------------------------------------------------------- GPU
@pytest.mark.gpu
def test_export_gpu_and_host_paths_give_the_same_bytes(gpu):
    from dimq_amd.export import assign_weight_indices, pack_indices, unpack_indices
    g = torch.Generator().manual_seed(8)
    for bits in (2, 3, 4, 8):
        announce(f"export paths bits={bits}")
        idx = torch.randint(0, 1 << bits, (12345,), generator=g, dtype=torch.uint8)
        host = pack_indices(idx, bits)
        dev = pack_indices(idx.to(gpu), bits)
        assert torch.equal(dev.cpu(), host)
        assert torch.equal(unpack_indices(dev, idx.numel(), bits).cpu(), unpack_indices(host, idx.numel(), bits))
    w = torch.randn(64, 40, generator=g)
    cb = torch.randn(16, generator=g).sort().values
    assert torch.equal(assign_weight_indices(w.to(gpu), cb.to(gpu)).cpu(), assign_weight_indices(w, cb))


@pytest.mark.gpu
@torch.no_grad()
def test_packed_checkpoint_resnet18_weight_only(gpu, tmp_path):
    """cfg3's mixed widths through the checkpoint: compact -> export (format 2) -> torch.load(weights_only)
    -> replace_modules_with_packed_dimq on a fresh ResNet-18 -> fp16 channels-last forward on the GPU,
    against the dequantized fp32 CPU model of the same checkpoint."""
    from dimq_amd.bench_models import resnet18
    from dimq_amd.export import export_packed_dimq_checkpoint, infer_module_hparams
    from dimq_amd.modules import DIMQCodebookConv2d, DIMQCodebookLinear, replace_modules_with_packed_dimq

    def pick(name, mod):
        if isinstance(mod, nn.Linear) or name == "conv1":
            return 8
        return 2 if mod.kernel_size == (3, 3) else 4

    announce("packed checkpoint resnet18")
    src = resnet18()
    compact = _compact(src, pick, per_channel=True)
    out = tmp_path / "resnet18_packed.pt"
    export_packed_dimq_checkpoint(compact, out, layer_hparams=infer_module_hparams(src))
    state = torch.load(out, map_location="cpu", weights_only=True)
    m = replace_modules_with_packed_dimq(resnet18(seed=99), state)
    convs = [x for x in m.modules() if isinstance(x, DIMQCodebookConv2d)]
    assert len(convs) == 20 and sum(isinstance(x, DIMQCodebookLinear) for x in m.modules()) == 1
    assert sorted({c.bits for c in convs}) == [2, 4, 8]
    for mod in m.modules():  # out_dtype of the runtime layers: the activations' dtype
        if isinstance(mod, (DIMQCodebookConv2d, DIMQCodebookLinear)):
            mod.out_dtype = torch.float16
    m = m.to(gpu).eval()
    x = torch.randn(2, 3, 64, 64, generator=torch.Generator().manual_seed(1))
    y = m(x.to(gpu).half().contiguous(memory_format=torch.channels_last)).float().cpu()
    ref = oracle.dequantized_model(m)(x)
    assert oracle.rel_err(y, ref) <= 1.5e-2, oracle.rel_err(y, ref)


@pytest.mark.gpu
@torch.no_grad()
def test_packed_checkpoint_w4a4_modules(gpu, tmp_path):
    """The reference format (16 per-layer centres, calibrated A4 qparams) through make_packed_layer:
    DIMQConv2d / DIMQLinear forwards against the oracle's LUT loops (reference.py:59-88,147-205)."""
    from dimq_amd.export import export_packed_dimq_checkpoint, infer_module_hparams
    from dimq_amd.modules import DIMQConv2d, DIMQLinear, make_packed_layer
    from tests.a4_check import a4_exact_check, a4_levels

    m = _net(3)
    compact = _compact(m, lambda n, mod: 4, per_channel=False)
    qp = {"conv1": {"scale": 0.125, "zero_point": 7}, "__default__": {"scale": 0.2, "zero_point": 8}}
    export_packed_dimq_checkpoint(compact, tmp_path / "a4.pt", act_qparams=qp, layer_hparams=infer_module_hparams(m))
    state = torch.load(tmp_path / "a4.pt", map_location="cpu", weights_only=True)
    g = torch.Generator().manual_seed(2)
    inputs = {"conv1": torch.randn(2, 3, 8, 8, generator=g), "conv2": torch.randn(2, 16, 8, 8, generator=g),
              "down": torch.randn(2, 16, 8, 8, generator=g), "fc": torch.randn(5, 512, generator=g)}
    for name, e in state["layers"].items():
        announce(f"w4a4 module {name}")
        mod = make_packed_layer(e).to(gpu)
        x = inputs[name]
        y = mod(x.to(gpu)).cpu()
        cb = e["codebook"].float()
        idx = torch.from_numpy(oracle.unpack_bits(e["packed_weight"].numpy(), e["weight_numel"], 4))
        bias = e["bias"].float()
        s, zp = e["act_scale"], e["act_zero_point"]
        if e["type"] == "linear":
            assert isinstance(mod, DIMQLinear)
            ref = oracle.linear_lut(x, e["packed_weight"], cb, s, zp, bias, e["out_features"], e["in_features"])
            exact = a4_levels(x, s, zp) @ cb.double()[idx.long()].reshape(e["weight_shape"]).T + bias.double()
            a4_exact_check(y, ref, exact, e["in_features"])
        else:
            assert isinstance(mod, DIMQConv2d)
            ref = oracle.conv2d_lut(x, e["packed_weight"], cb, s, zp, bias, e["weight_shape"], e["stride"],
                                    e["padding"], e["dilation"], e["groups"])
            w_hat = cb.double()[idx.long()].reshape(e["weight_shape"])
            exact = torch.nn.functional.conv2d(a4_levels(x, s, zp), w_hat, bias.double(), e["stride"], e["padding"],
                                               e["dilation"], e["groups"])
            a4_exact_check(y, ref, exact, int(np.prod(e["weight_shape"][1:])))


@pytest.mark.gpu
@torch.no_grad()
def test_prepared_conv_weight_follows_load_state_dict(gpu):
    """DIMQCodebookConv2d caches its kernel-layout weight; load_state_dict (an in-place copy into the same
    buffer) must invalidate it."""
    from dimq_amd.modules import DIMQCodebookConv2d
    announce("prepared weight after load_state_dict")
    g = torch.Generator().manual_seed(12)
    convs = [nn.Conv2d(64, 64, 3, 1, 1) for _ in range(2)]
    for c in convs:
        c.weight.data = torch.randn(64, 64, 3, 3, generator=g) * 0.05
    a = DIMQCodebookConv2d.from_conv(convs[0].to(gpu), 2, out_dtype=torch.float32)
    b = DIMQCodebookConv2d.from_conv(convs[1].to(gpu), 2, out_dtype=torch.float32)
    x = torch.randn(2, 64, 16, 16, generator=g).half()
    ya = a(x.to(gpu))
    ptr = a.packed_weight.data_ptr()
    a.load_state_dict(b.state_dict())
    assert a.packed_weight.data_ptr() == ptr  # copied in place: the cache key by address alone would be stale
    y = a(x.to(gpu))
    ref = oracle.conv2d_dequant_reference(x.float(), b.packed_weight.cpu(), 2, b.codebook.cpu(), (64, 64, 3, 3),
                                          b.bias.cpu(), 1, 1, 1, 1)
    assert oracle.rel_err(y, ref) <= 2e-3
    assert oracle.rel_err(ya, ref) > 0.1  # the two layers differ
