"""The pre-decoded-weight Linear path (M >= 2048): the weights decoded once per
call into the workspace as fp16 (bf16 / fp32 activations converted to fp16
there too, with per-row range flags), then an fp16 GEMM fed by
global_load_lds.  Checked against dequantize-then-F.linear in fp32 on the CPU
(reference.py:91-110, oracle.linear_dequant_reference) at the weight-only bar
2e-3 (bf16 outputs 8e-3), over bit widths, per-layer and per-output-channel
codebooks, activation dtypes, ragged M / N tails, K not a multiple of 64,
each tile shape and every fused epilogue the path instantiates."""

from __future__ import annotations

import pytest
import torch

import oracle
from tests.conftest import announce, out_tol

pytestmark = pytest.mark.gpu


def _case(M, N, K, bits, per_channel, seed, xdt=torch.float16):
    g = torch.Generator().manual_seed(seed)
    E = 1 << bits
    rows = N if per_channel else 1
    cb = (torch.randn(rows, E, generator=g) * 0.05).sort(dim=1).values
    idx = torch.randint(0, E, (N, K), generator=g, dtype=torch.uint8)
    packed = torch.from_numpy(oracle.pack_bits(idx, bits))
    x = torch.randn(M, K, generator=g).to(xdt)
    bias = torch.randn(N, generator=g) * 0.05
    return cb, packed, x, bias


def test_workspace_query_selects_the_path():
    from dimq_amd import _C
    lib = _C.lib
    F32, F16, BF16, F64 = 0, 1, 2, 3
    assert lib.dimq_linear_codebook_workspace_bytes(12608, 768, 3072, 4, F16) >= 3072 * 768 * 2 + 3072 * 4
    assert lib.dimq_linear_codebook_workspace_bytes(2048, 96, 352, 3, F16) >= 352 * 96 * 2 + 352 * 4
    # bf16 / fp32 activations also keep their fp16 copy and one flag per row
    assert lib.dimq_linear_codebook_workspace_bytes(2048, 768, 3072, 4, F32) >= \
        3072 * 768 * 2 + 3072 * 4 + 2048 * 768 * 2 + 2048 * 4
    assert lib.dimq_linear_codebook_workspace_bytes(12608, 768, 768, 4, BF16) >= \
        768 * 768 * 2 + 768 * 4 + 12608 * 768 * 2 + 12608 * 4
    assert lib.dimq_linear_codebook_workspace_bytes(2047, 768, 3072, 4, F16) == 0  # below the M threshold
    assert lib.dimq_linear_codebook_workspace_bytes(1576, 768, 3072, 4, F32) == 0  # cfg1: the fused deep tile
    assert lib.dimq_linear_codebook_workspace_bytes(12608, 768, 3072, 4, F64) == 0
    assert lib.dimq_linear_codebook_workspace_bytes(12608, 80, 3072, 4, F16) == 0  # K % 32 != 0
    assert lib.dimq_linear_codebook_workspace_bytes(12608, 768, 3072, 8, F16) == 0


@pytest.mark.parametrize("xdt", [torch.float16, torch.bfloat16, torch.float32])
@pytest.mark.parametrize("bits", [2, 3, 4])
@pytest.mark.parametrize("per_channel", [True, False])
@torch.no_grad()
def test_predecoded_linear_vs_dequant_reference(gpu, bits, per_channel, xdt):
    from dimq_amd import ops
    M, N, K = 2085, 352, 96  # tails: M % 256 = 37, N % 256 = 96, K % 64 = 32
    announce(f"predecode bits={bits} per_channel={per_channel} x={xdt} M={M} N={N} K={K}")
    cb, packed, x, bias = _case(M, N, K, bits, per_channel, 10 * bits + per_channel, xdt)
    y = ops.dimq_linear_codebook(x.to(gpu), packed.to(gpu), cb.to(gpu), bits, bias.to(gpu), N, K,
                                 out_dtype=torch.float32)
    ref = oracle.linear_dequant_reference(x.float(), packed, bits, cb, N, K, bias)
    assert oracle.rel_err(y.cpu(), ref) <= 2e-3


@pytest.mark.parametrize("M,N,K", [(2304, 512, 256), (2200, 768, 64), (8704, 2048, 32), (8192, 1024, 64),
                                   (8192, 1024, 96), (8192, 128, 64), (4200, 768, 192), (4100, 512, 1024)])
# tiles 3, 2, 1, 0; K % 64 = 32 moves tile 0's shape to 1; N <= 128 takes tile 3; the last two take tile 4
# (160 x 256, ragged M: 4200 % 160 = 40, 4100 % 160 = 100)
@pytest.mark.parametrize("epi,out,xdt", [("relu", torch.float32, torch.float16), ("gelu", torch.float16, torch.float16),
                                         ("residual", torch.bfloat16, torch.float16), (None, torch.bfloat16, torch.float16),
                                         ("residual", torch.bfloat16, torch.bfloat16), (None, torch.float32, torch.float32)])
@torch.no_grad()
def test_predecoded_linear_epilogues(gpu, M, N, K, epi, out, xdt):
    from dimq_amd import ops
    announce(f"predecode epilogue={epi} out={out} x={xdt} M={M} N={N} K={K}")
    cb, packed, x, bias = _case(M, N, K, 4, True, 7, xdt)
    res = (torch.randn(M, N, generator=torch.Generator().manual_seed(8)) * 0.5).bfloat16() \
        if epi == "residual" else None
    y = ops.dimq_linear_codebook(x.to(gpu), packed.to(gpu), cb.to(gpu), 4, bias.to(gpu), N, K, out_dtype=out,
                                 residual=None if res is None else res.to(gpu),
                                 activation=epi if epi in ("relu", "gelu") else None)
    ref = oracle.linear_dequant_reference(x.float(), packed, 4, cb, N, K, bias)
    if epi == "residual":
        ref = ref + res.float()
    elif epi == "gelu":
        ref = torch.nn.functional.gelu(ref)
    elif epi == "relu":
        ref = torch.relu(ref)
    tol = out_tol(out)
    assert oracle.rel_err(y.float().cpu(), ref) <= tol


@torch.no_grad()
def test_predecoded_small_centres_keep_precision(gpu):
    """Per-channel centres around 1e-6 (fp16 subnormals unscaled): the per-row power-of-two scaling of the
    decoded rows keeps 11 significant bits."""
    from dimq_amd import ops
    M, N, K = 2048, 256, 128
    announce("predecode tiny centres")
    cb, packed, x, bias = _case(M, N, K, 4, True, 11)
    cb = cb * 2e-5
    y = ops.dimq_linear_codebook(x.to(gpu), packed.to(gpu), cb.to(gpu), 4, None, N, K, out_dtype=torch.float32)
    ref = oracle.linear_dequant_reference(x.float(), packed, 4, cb, N, K, None)
    assert oracle.rel_err(y.cpu(), ref) <= 2e-3


@torch.no_grad()
def test_predecoded_matches_fused_path(gpu):
    """The same call with and without a workspace (the fused shared-decode tile): both within the bar of the
    oracle and of each other."""
    from dimq_amd import _C, ops
    M, N, K = 4096, 768, 768
    announce("predecode vs fused")
    cb, packed, x, bias = _case(M, N, K, 4, True, 12)
    xg, pg, cg, bg = x.to(gpu), packed.to(gpu), cb.to(gpu), bias.to(gpu)
    y_pd = ops.dimq_linear_codebook(xg, pg, cg, 4, bg, N, K, out_dtype=torch.float32)
    y_fu = torch.empty_like(y_pd)
    with torch.cuda.device(gpu):
        rc = _C.lib.dimq_linear_codebook(xg.data_ptr(), 1, M, K, pg.data_ptr(), pg.numel(), 4, cg.data_ptr(), 0, N,
                                         16, bg.data_ptr(), 0, N, y_fu.data_ptr(), 0, 0,
                                         torch.cuda.current_stream().cuda_stream)
    assert rc == 0
    ref = oracle.linear_dequant_reference(x.float(), packed, 4, cb, N, K, bias)
    assert oracle.rel_err(y_pd.cpu(), ref) <= 2e-3
    assert oracle.rel_err(y_fu.cpu(), ref) <= 2e-3
    assert oracle.rel_err(y_pd.cpu(), y_fu.cpu()) <= 2e-3


# ---------------------------------------------------------------- batched weight pre-decode
@pytest.mark.parametrize("xdt", [torch.float16, torch.bfloat16, torch.float32])
@torch.no_grad()
def test_predecode_batch_matches_per_call_decode(gpu, xdt):
    """dimq_codebook_predecode_batch over 38 layers (2, 3 and 4 bits, per-layer and per-channel codebooks,
    more than one launch's 32 jobs): each layer's Linear on its batch decode gives the same bits as the same
    call decoding its own weights (same decode, same GEMM), and stays within the bar of the oracle."""
    from dimq_amd import ops
    M = 2048
    announce(f"predecode batch x={xdt}")
    shapes = [(64, 64, 2 + i % 3, i % 2 == 0) for i in range(34)] + [(352, 96, 3, True), (768, 256, 4, False),
                                                                      (256, 512, 2, True), (512, 64, 4, True)]
    layers, cases = [], []
    for i, (N, K, bits, pc) in enumerate(shapes):
        cb, packed, x, bias = _case(M, N, K, bits, pc, 100 + i, xdt)
        cases.append((cb, packed, x, bias, N, K, bits))
        layers.append((packed.to(gpu), cb.to(gpu), bits, N, K))
    buf, views = ops.predecode_codebook_weights(layers)
    assert all(v is not None for v in views) and buf is not None
    for i, ((cb, packed, x, bias, N, K, bits), (pg, cg, _, _, _)) in enumerate(zip(cases, layers)):
        xg, bg = x.to(gpu), bias.to(gpu)
        y_own = ops.dimq_linear_codebook(xg, pg, cg, bits, bg, N, K, out_dtype=torch.float32)
        y_bat = ops.dimq_linear_codebook(xg, pg, cg, bits, bg, N, K, out_dtype=torch.float32, decoded=views[i])
        assert torch.equal(y_own, y_bat), (i, N, K, bits)
        if i in (0, 1, 2, 34, 35, 36, 37):
            ref = oracle.linear_dequant_reference(x.float(), packed, bits, cb, N, K, bias)
            assert oracle.rel_err(y_bat.cpu(), ref) <= 2e-3, (i, N, K, bits)


def _scaled_decode_cpu(packed, bits, cb, N, K):
    """The decode's contract on the CPU: W_hat[n] = fp16(C[idx] * 2^e_n) (round to nearest even), with e_n =
    clamp(15 - ex, -100, 100) for max|C_n| = m * 2^ex, m in [0.5, 1) (e_n = 0 for an all-zero row), and the
    row factor 2^-e_n; C[idx] from the oracle's dequantize (reference.py:47-56)."""
    import numpy as np
    w = oracle.dequantize(packed, bits, cb, N, K).astype(np.float32)
    c = cb.float().numpy().reshape(-1 if cb.shape[0] != 1 else 1, cb.shape[-1])
    mx = np.abs(c).max(axis=1)
    ex = np.frexp(mx)[1]
    e = np.where(mx > 0, np.clip(15 - ex, -100, 100), 0).astype(np.int32)
    e = np.broadcast_to(e, (N,)) if e.shape[0] == 1 else e
    w_hat = np.ldexp(w, e[:, None]).astype(np.float32).astype(np.float16)
    return w_hat, np.ldexp(np.float32(1.0), -e).astype(np.float32)


@torch.no_grad()
def test_predecode_batch_is_the_scaled_dequantized_weight(gpu):
    """The decoded fp16 rows and their factors, bit for bit, against the CPU statement of the decode: 2, 3 and
    4 bits, per-layer and per-channel codebooks, a codebook with fewer entries than 2^bits, an all-zero row,
    centres near fp16's subnormals and near its largest values (the exponent clamp), K past one lane pass."""
    import numpy as np
    from dimq_amd import ops
    announce("predecode decode bits")
    cases = []
    for i, (N, K, bits, rows, size) in enumerate([(37, 64, 2, 37, 4), (64, 96, 3, 1, 8), (130, 768, 4, 130, 16),
                                                  (16, 4608, 4, 16, 16), (33, 128, 4, 33, 10), (24, 3072, 3, 24, 8)]):
        g = torch.Generator().manual_seed(300 + i)
        cb = (torch.randn(rows, size, generator=g) * 0.05).sort(dim=1).values
        if rows > 2:
            cb[0] = 0.0                   # all-zero row: e = 0
            cb[1] *= 1e-30                # e clamped at +100
            cb[2] = cb[2] * 1e4           # largest entries near 2^15 after scaling
        idx = torch.randint(0, size, (N, K), generator=g, dtype=torch.uint8)
        packed = torch.from_numpy(oracle.pack_bits(idx, bits))
        cases.append((packed, cb, bits, N, K))
    layers = [(p.to(gpu), c.to(gpu), b, n, k) for p, c, b, n, k in cases]
    buf, views = ops.predecode_codebook_weights(layers)
    for (packed, cb, bits, N, K), v in zip(cases, views):
        got = v.cpu().numpy()
        w_gpu = got[: N * K * 2].view(np.float16).reshape(N, K)
        off = (N * K * 2 + 255) // 256 * 256
        rs_gpu = got[off: off + 4 * N].view(np.float32)
        w_ref, rs_ref = _scaled_decode_cpu(packed, bits, cb, N, K)
        assert np.array_equal(w_gpu.view(np.uint16), w_ref.view(np.uint16)), (N, K, bits)
        assert np.array_equal(rs_gpu, rs_ref), (N, K, bits)


@torch.no_grad()
def test_predecode_batch_epilogues_and_small_m(gpu):
    """Fused residual / GELU epilogues on decoded weights; a call below the large-M threshold ignores `decoded`
    and decodes per call as before; layers the batch cannot decode (8 bits, K % 32 != 0) get no view."""
    from dimq_amd import ops
    announce("predecode batch epilogues")
    M, N, K = 4200, 768, 192
    cb, packed, x, bias = _case(M, N, K, 4, True, 41)
    pg, cg, xg, bg = packed.to(gpu), cb.to(gpu), x.to(gpu), bias.to(gpu)
    cb8 = (torch.randn(N, 256) * 0.05).sort(dim=1).values.to(gpu)
    p8 = torch.randint(0, 256, (N * K,), dtype=torch.uint8).to(gpu)
    p80 = torch.from_numpy(oracle.pack_bits(torch.randint(0, 16, (N, 80), dtype=torch.uint8), 4)).to(gpu)
    _, views = ops.predecode_codebook_weights([(pg, cg, 4, N, K), (p8, cb8, 8, N, K), (p80, cg, 4, N, 80)])
    assert views[0] is not None and views[1] is None and views[2] is None
    res = (torch.randn(M, N, generator=torch.Generator().manual_seed(42)) * 0.5).bfloat16().to(gpu)
    for kw in ({"residual": res}, {"activation": "gelu"}):
        a = ops.dimq_linear_codebook(xg, pg, cg, 4, bg, N, K, out_dtype=torch.bfloat16, **kw)
        b = ops.dimq_linear_codebook(xg, pg, cg, 4, bg, N, K, out_dtype=torch.bfloat16, decoded=views[0], **kw)
        assert torch.equal(a, b), kw
    small = xg[:100]
    a = ops.dimq_linear_codebook(small, pg, cg, 4, bg, N, K, out_dtype=torch.float32)
    b = ops.dimq_linear_codebook(small, pg, cg, 4, bg, N, K, out_dtype=torch.float32, decoded=views[0])
    assert torch.equal(a, b)
    with pytest.raises(RuntimeError, match="decoded"):
        ops.dimq_linear_codebook(xg, pg, cg, 4, bg, N, K, decoded=views[0][:1000])


@torch.no_grad()
def test_decoded_weights_context_in_a_model(gpu):
    """modules.decoded_weights: the ViT blocks' codebook Linears run on one batch decode per forward, with the
    same outputs as per-call decoding, and the views are dropped when the block ends."""
    from dimq_amd.bench_models import quantize_vit, ViT
    from dimq_amd.modules import DIMQCodebookLinear, decoded_weights
    announce("decoded_weights ViT-small M=2 x 1025")
    torch.manual_seed(1)
    m = ViT(image=256, patch=8, dim=128, depth=2, heads=4, mlp=256, classes=10)   # 32x32 patches + cls: 1025 tokens
    for mod in m.modules():
        if isinstance(mod, torch.nn.Linear):
            torch.nn.init.normal_(mod.weight, std=0.02)
    from tests.test_gpu_models import _cast_float_params
    m = _cast_float_params(quantize_vit(m.to(gpu), 4, out_dtype=torch.bfloat16), torch.bfloat16).eval()
    x = torch.randn(2, 3, 256, 256, device=gpu).bfloat16()
    y_ctx = m(x)                                             # forward uses decoded_weights (M = 2050 rows)
    lin = [mod for mod in m.modules() if isinstance(mod, DIMQCodebookLinear)]
    assert all(mod._decoded is None for mod in lin)
    h = m.embed(x)
    h = torch.cat([m.class_token.expand(2, -1, -1), h], dim=1) + m.pos_embedding
    with decoded_weights(m, h.shape[0] * h.shape[1]):
        assert sum(mod._decoded is not None for mod in lin) == 8
    for blk in m.blocks:
        h = blk(h)
    y_own = m.head(m.ln(h[:, 0]))
    assert torch.equal(y_ctx, y_own)


@torch.no_grad()
def test_predecoded_paths_under_graph_replay(gpu):
    """The pre-decoded Linear (fp16 x; bf16 x with its conversion and range flags; GELU) and the batched
    decode captured in a HIP graph: every replay, with unrelated eager work between replays, gives the eager
    result bit for bit (bench.py times these paths as graph replays)."""
    from dimq_amd import ops
    announce("predecode graph replay M=2304")
    M, N, K = 2304, 512, 256
    cb, packed, x, bias = _case(M, N, K, 4, True, 77)
    pg, cg, bg, xg = packed.to(gpu), cb.to(gpu), bias.to(gpu), x.to(gpu)
    xbg = x.bfloat16().to(gpu)

    def run():
        y1 = ops.dimq_linear_codebook(xg, pg, cg, 4, bg, N, K, out_dtype=torch.float32)
        y2 = ops.dimq_linear_codebook(xbg, pg, cg, 4, bg, N, K, out_dtype=torch.bfloat16, activation="gelu")
        _, views = ops.predecode_codebook_weights([(pg, cg, 4, N, K)])
        y3 = ops.dimq_linear_codebook(xg, pg, cg, 4, bg, N, K, out_dtype=torch.float32, decoded=views[0])
        return y1, y2, y3

    eager = run()
    assert torch.equal(eager[0], eager[2])
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        run()
    torch.cuda.current_stream().wait_stream(s)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        outs = run()
    for r in range(3):
        for o in outs:
            o.zero_()
        _ = (xg * 2).sum()  # unrelated eager work between replays
        graph.replay()
        torch.cuda.synchronize()
        for o, e in zip(outs, eager):
            assert torch.equal(o, e), f"replay {r}"
